"""Pins of the CPU oracle (oracle/lstm_oracle.c) -- the checker every GPU parity test relies on.

The reference ships no golden vectors for this path, so the oracle is pinned by:
  * torch's fp32 CPU nn.LSTM / nn.Linear (the library routine the reference's CPU path restates,
    persistent_lstm_reference.cpp:7-64), including packed sequences and initial states;
  * the reference's own CPU path compiled from its sources into oracle/_ref (when built);
  * closed forms: zero weights reduce the recurrence to scalar maps that are solved here directly;
  * brute force with a tiny hand-written recurrence on H = 1;
  * planted mistakes: each mutation of the oracle must be caught by the torch comparison.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import linear_params, make_regressor, make_x, oracle_layers
from oracle import oracle


def _torch_lstm(I, H, L, seed=0, bias=True):
    torch.manual_seed(seed)
    return torch.nn.LSTM(I, H, L, batch_first=True, bias=bias).eval()


@pytest.mark.parametrize("I,H,L,B,T", [(5, 128, 1, 8, 64), (7, 16, 3, 5, 23), (3, 9, 2, 4, 1), (1, 1, 4, 2, 17)])
def test_lstm_matches_torch(I, H, L, B, T):
    lstm = _torch_lstm(I, H, L)
    x = make_x(B, T, I)
    with torch.inference_mode():
        out, (h, c) = lstm(x)
    r = oracle.lstm_forward(x.numpy(), oracle_layers(lstm), want_seq=True)
    np.testing.assert_allclose(r["out_seq"], out.numpy(), atol=2e-6)
    np.testing.assert_allclose(r["h_n"], h.numpy(), atol=2e-6)
    np.testing.assert_allclose(r["c_n"], c.numpy(), atol=2e-6)


def test_regressor_matches_torch_c1():
    native = make_regressor(5, 128, 1, 24)
    x = make_x(8, 64, 5)
    with torch.inference_mode():
        want = native(x).numpy()
    got = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear))
    np.testing.assert_allclose(got, want, atol=2e-6)


def test_initial_state_matches_torch():
    I, H, L, B, T = 4, 12, 2, 3, 15
    lstm = _torch_lstm(I, H, L, seed=3)
    x = make_x(B, T, I)
    g = torch.Generator().manual_seed(11)
    h0, c0 = torch.randn(L, B, H, generator=g), torch.randn(L, B, H, generator=g)
    with torch.inference_mode():
        out, (h, c) = lstm(x, (h0, c0))
    r = oracle.lstm_forward(x.numpy(), oracle_layers(lstm), h0=h0.numpy(), c0=c0.numpy(), want_seq=True)
    np.testing.assert_allclose(r["out_seq"], out.numpy(), atol=2e-6)
    np.testing.assert_allclose(r["h_n"], h.numpy(), atol=2e-6)
    np.testing.assert_allclose(r["c_n"], c.numpy(), atol=2e-6)


def test_probes_equal_prefix_runs():
    """The state after p steps equals the final state of a run on x[:, :p]."""
    I, H, L, B, T = 5, 24, 3, 4, 40
    lstm = _torch_lstm(I, H, L, seed=5)
    x = make_x(B, T, I)
    steps = (1, 7, 40)
    r = oracle.lstm_forward(x.numpy(), oracle_layers(lstm), probe_steps=steps)
    for p, t in enumerate(steps):
        with torch.inference_mode():
            _, (h, c) = lstm(x[:, :t])
        np.testing.assert_allclose(r["probe_h"][p], h.numpy(), atol=2e-6)
        np.testing.assert_allclose(r["probe_c"][p], c.numpy(), atol=2e-6)


@pytest.mark.parametrize("sort", [True, False])
def test_ragged_matches_packed_sequence(sort):
    I, H, L, B, T = 5, 20, 2, 7, 30
    lstm = _torch_lstm(I, H, L, seed=7)
    x = make_x(B, T, I)
    lengths = torch.randint(1, T + 1, (B,), generator=torch.Generator().manual_seed(2))
    if sort:
        lengths = torch.sort(lengths, descending=True).values
    packed = torch.nn.utils.rnn.pack_padded_sequence(x, lengths, batch_first=True, enforce_sorted=sort)
    with torch.inference_mode():
        po, (h, c) = lstm(packed)
    out, _ = torch.nn.utils.rnn.pad_packed_sequence(po, batch_first=True, total_length=T)
    r = oracle.lstm_forward(x.numpy(), oracle_layers(lstm), lengths=lengths.numpy(), want_seq=True)
    np.testing.assert_allclose(r["out_seq"], out.numpy(), atol=2e-6)
    np.testing.assert_allclose(r["h_n"], h.numpy(), atol=2e-6)
    np.testing.assert_allclose(r["c_n"], c.numpy(), atol=2e-6)


def test_zero_weights_closed_form():
    """W = 0: gates are constants sigma(b) / tanh(b); c_t = s_f c_{t-1} + s_i tanh(b_g), h_t = s_o tanh(c_t)."""
    I, H, L, B, T = 3, 6, 2, 2, 25
    rng = np.random.default_rng(0)
    layers = []
    for l in range(L):
        K = I if l == 0 else H
        b_ih = rng.normal(size=4 * H).astype(np.float32)
        b_hh = rng.normal(size=4 * H).astype(np.float32)
        layers.append((np.zeros((4 * H, K), np.float32), np.zeros((4 * H, H), np.float32), b_ih, b_hh))
    x = rng.normal(size=(B, T, I)).astype(np.float32)
    c0 = rng.normal(size=(L, B, H)).astype(np.float32)
    r = oracle.lstm_forward(x, layers, c0=c0, h0=np.zeros((L, B, H), np.float32))
    sig = lambda v: 1.0 / (1.0 + math.exp(-v))  # noqa: E731
    for l, (_, _, bi, bh) in enumerate(layers):
        for u in range(H):
            b = [float(bi[g * H + u]) + float(bh[g * H + u]) for g in range(4)]
            for bb in range(B):
                c = float(c0[l, bb, u])
                for _ in range(T):
                    c = sig(b[1]) * c + sig(b[0]) * math.tanh(b[2])
                h = sig(b[3]) * math.tanh(c)
                assert abs(r["c_n"][l, bb, u] - c) < 1e-6
                assert abs(r["h_n"][l, bb, u] - h) < 1e-6


def test_zero_everything_decays():
    """W = 0 and b = 0: every gate is 1/2 and g = 0, so c_t = c0 / 2^t and h_t = tanh(c_t) / 2."""
    H, T = 5, 12
    layers = [(np.zeros((4 * H, 2), np.float32), np.zeros((4 * H, H), np.float32), None, None)]
    c0 = np.full((1, 1, H), 3.0, np.float32)
    r = oracle.lstm_forward(np.ones((1, T, 2), np.float32), layers, c0=c0, probe_steps=(1, T))
    assert np.allclose(r["probe_c"][0], 1.5) and np.allclose(r["probe_c"][1], 3.0 / 2 ** T)
    assert np.allclose(r["h_n"], 0.5 * np.tanh(3.0 / 2 ** T))


def test_scalar_brute_force():
    """H = 1, I = 1: the recurrence written out by hand."""
    rng = np.random.default_rng(1)
    w_ih = rng.normal(size=(4, 1)).astype(np.float32)
    w_hh = rng.normal(size=(4, 1)).astype(np.float32)
    b_ih = rng.normal(size=4).astype(np.float32)
    b_hh = rng.normal(size=4).astype(np.float32)
    xs = rng.normal(size=(1, 9, 1)).astype(np.float32)
    r = oracle.lstm_forward(xs, [(w_ih, w_hh, b_ih, b_hh)])
    h = c = 0.0
    s = lambda v: 1 / (1 + math.exp(-v))  # noqa: E731
    for t in range(9):
        z = [float(w_ih[g, 0]) * float(xs[0, t, 0]) + float(b_ih[g]) + float(w_hh[g, 0]) * h + float(b_hh[g])
             for g in range(4)]
        c = s(z[1]) * c + s(z[0]) * math.tanh(z[2])
        h = s(z[3]) * math.tanh(c)
    assert abs(r["h_n"][0, 0, 0] - h) < 1e-6 and abs(r["c_n"][0, 0, 0] - c) < 1e-6


def test_row_permutation_equivariance():
    lstm = _torch_lstm(5, 16, 2, seed=9)
    x = make_x(6, 20, 5)
    perm = np.array([3, 0, 5, 1, 4, 2])
    a = oracle.lstm_forward(x.numpy(), oracle_layers(lstm))["h_n"]
    b = oracle.lstm_forward(x.numpy()[perm], oracle_layers(lstm))["h_n"]
    np.testing.assert_array_equal(a[:, perm], b)


@pytest.mark.parametrize("mutation", [m for m in oracle.MUTATIONS if m != "none"])
def test_planted_mistakes_are_caught(mutation):
    """Every plausible slip (gate order, dropped term, transposed operand, missing nonlinearity)
    moves the result far outside the comparison tolerance against torch."""
    lstm = _torch_lstm(5, 16, 2, seed=13)
    x = make_x(4, 30, 5)
    with torch.inference_mode():
        want = lstm(x)[0].numpy()
    good = oracle.lstm_forward(x.numpy(), oracle_layers(lstm), want_seq=True)["out_seq"]
    bad = oracle.lstm_forward(x.numpy(), oracle_layers(lstm), want_seq=True, mutation=mutation)["out_seq"]
    assert np.abs(good - want).max() < 2e-6
    assert np.abs(bad - want).max() > 1e-2, f"mutation {mutation} not detected"


def test_half_conversion_matches_numpy():
    # every finite half value round-trips, and random floats round like numpy's float16
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    halfs = bits.view(np.float16)
    finite = np.isfinite(halfs)
    vals = halfs[finite].astype(np.float32)
    np.testing.assert_array_equal(oracle.round_half(vals), vals)
    rng = np.random.default_rng(3)
    v = (rng.normal(size=200000) * 10.0 ** rng.integers(-9, 6, size=200000)).astype(np.float32)
    ties = (np.arange(-3000, 3000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10)  # halfway cases
    for arr in (v, ties, np.float32([65504, 65519.99, 65520, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25])):
        np.testing.assert_array_equal(oracle.round_half(arr), arr.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("mode", ["ref_fp16", "ref_fp16_proj"])
def test_ref_fp16_modes_match_stepwise_torch_emulation(mode):
    """numerics='ref_fp16' (fp16-rounded fused bias and h, fp32 c) and 'ref_fp16_proj' (plus the
    fp16-rounded input projection) against an independent torch LSTMCell loop that rounds the same
    quantities.  With I = 40 inputs of magnitude ~1 the projection rounding moves gates by ~1e-3, so
    dropping it (or applying it in the wrong mode) fails the c bound."""
    I, H, B, T = 40, 32, 3, 40
    lstm = _torch_lstm(I, H, 1, seed=21)
    x = make_x(B, T, I).half().float()
    w_ih, w_hh, b_ih, b_hh = (getattr(lstm, f"{n}_l0").detach().half().float()
                              for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"))
    bias = (b_ih + b_hh).half().float()
    h = torch.zeros(B, H)
    c = torch.zeros(B, H)
    for t in range(T):
        p = x[:, t].double() @ w_ih.double().t()
        if mode == "ref_fp16_proj":
            p = p.float().half().double()
        z = p + h.double() @ w_hh.double().t() + bias.double()
        i, f, g, o = z.chunk(4, dim=1)
        c = (torch.sigmoid(f) * c.double() + torch.sigmoid(i) * torch.tanh(g)).float()
        h = (torch.sigmoid(o) * torch.tanh(c.double())).float().half().float()
    layers = [tuple(t.numpy() for t in (w_ih, w_hh, b_ih, b_hh))]
    r = oracle.lstm_forward(x.numpy(), layers, numerics=mode)
    np.testing.assert_allclose(r["h_n"][0], h.numpy(), atol=1e-3)
    np.testing.assert_allclose(r["c_n"][0], c.numpy(), atol=1e-5)
    assert np.abs(r["h_n"][0] - h.numpy()).mean() < 1e-5
    other = oracle.lstm_forward(x.numpy(), layers, numerics="ref_fp16_proj" if mode == "ref_fp16" else "ref_fp16")
    assert np.abs(other["c_n"][0] - c.numpy()).max() > 1e-5, "the two modes must differ measurably"


def test_ref_fp16_proj_l1_rounds_only_the_hidden_layers_projections():
    """numerics='ref_fp16_proj_l1' (layer 0's projection unrounded, layers >= 1 rounded): layer 0 is
    exactly ref_fp16's layer 0, and layer 1 is exactly a one-layer ref_fp16_proj run over layer 0's
    fp16 output sequence."""
    I, H, B, T = 7, 24, 3, 30
    lstm = _torch_lstm(I, H, 2, seed=23)
    x = make_x(B, T, I).numpy()
    layers = [tuple(getattr(lstm, f"{n}_l{l}").detach().numpy() for n in ("weight_ih", "weight_hh", "bias_ih",
                                                                            "bias_hh")) for l in range(2)]
    both = oracle.lstm_forward(x, layers, numerics="ref_fp16_proj_l1", probe_steps=(1, T))
    first = oracle.lstm_forward(x, layers[:1], numerics="ref_fp16", probe_steps=(1, T), want_seq=True)
    np.testing.assert_array_equal(both["probe_h"][:, 0], first["probe_h"][:, 0])
    np.testing.assert_array_equal(both["probe_c"][:, 0], first["probe_c"][:, 0])
    second = oracle.lstm_forward(first["out_seq"], layers[1:], numerics="ref_fp16_proj", probe_steps=(1, T))
    np.testing.assert_array_equal(both["probe_h"][:, 1], second["probe_h"][:, 0])
    np.testing.assert_array_equal(both["probe_c"][:, 1], second["probe_c"][:, 0])
    # and it is neither of the uniform modes
    for other in ("ref_fp16", "ref_fp16_proj"):
        r = oracle.lstm_forward(x, layers, numerics=other, probe_steps=(1, T))
        assert not np.array_equal(r["probe_c"], both["probe_c"]), other


def test_linear_modes_match_float64():
    """oracle.linear: fp32 mode = float64 product rounded to float32; ref_fp16 = operands rounded to
    fp16, float64 product rounded through float32 to fp16 (the reference head's fp16 output)."""
    rng = np.random.default_rng(9)
    inp = rng.normal(size=(7, 33)).astype(np.float32)
    w = (rng.normal(size=(5, 33)) / 4).astype(np.float32)
    b = rng.normal(size=5).astype(np.float32)
    want32 = (inp.astype(np.float64) @ w.T.astype(np.float64) + b).astype(np.float32)
    np.testing.assert_array_equal(oracle.linear(inp, w, b), want32)
    h = lambda a: a.astype(np.float16).astype(np.float64)  # noqa: E731
    want16 = (h(inp) @ h(w).T + h(b)).astype(np.float32).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(oracle.linear(inp, w, b, numerics="ref_fp16"), want16)
    assert not np.array_equal(oracle.linear(inp, w, b, numerics="ref_fp16"), want32)


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (needs the reference checkout)")
def test_reference_cpu_path_agrees_with_oracle():
    native = make_regressor(5, 32, 4, 6, seed=17)
    x = make_x(6, 50, 5)
    layers = oracle_layers(native.lstm)
    lw, lb = linear_params(native.linear)
    ours = oracle.regressor_forward(x.numpy(), layers, lw, lb)
    theirs = oracle.ref_regressor_forward(x.numpy(), layers, lw, lb, threads=2)
    np.testing.assert_allclose(ours, theirs, atol=2e-6)
