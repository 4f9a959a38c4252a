"""The reference's extension entry points (bindings.cpp:154-165), each fed the reference's own
argument formats, against the CPU oracle; and the uniform-batch cache against allocator reuse.

Formats restated from the reference (test code, not product code):
  kpairs   P[p, c, j] = W[c, 2p + j], zero-padded to even K          model.py:20-27
  fused    bias_ih + bias_hh summed in the model's dtype (fp16)       model.py:552
  packed   W^T [K, 4H] contiguous                                      persistent_lstm_hip.cu:2005-2018
  uniform  (x[0:1], virtual_batch_size, *projected_args) -> [1, O]    model.py:628-645
The oracle gets exactly the fp16 values the GPU gets (weights, fused bias, x), so the only
differences are accumulation order, transcendental rounding and the fp16 h of every step.  Two
bounds: the north-star tolerance against the fp32 oracle, and a regression bound against the
oracle's `ref_fp16` mode, which restates that per-step rounding.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import persistent_lstm_hip_ext as ext_mod
from conftest import assert_close, make_regressor, make_x
from oracle import oracle
from persistent_lstm_hip_amd import PersistentLSTMRegressor

pytestmark = pytest.mark.gpu

REGRESSION_MAX_ABS = 1e-3
REGRESSION_MEAN_ABS = 1e-4


def _say(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def kpairs(w: torch.Tensor) -> torch.Tensor:
    k = w.shape[1]
    wt = torch.nn.functional.pad(w.t(), (0, 0, 0, k % 2))
    return wt.reshape(-1, 2, w.shape[0]).permute(0, 2, 1).contiguous()


@pytest.fixture(scope="module")
def setup():
    I, H, L, O, B, T = 5, 128, 4, 24, 40, 70
    native = make_regressor(I, H, L, O).half()
    lstm = native.lstm
    dev = torch.device("cuda")
    w_ih = [getattr(lstm, f"weight_ih_l{l}").detach().to(dev) for l in range(L)]
    w_hh = [getattr(lstm, f"weight_hh_l{l}").detach().to(dev) for l in range(L)]
    fused = [(getattr(lstm, f"bias_ih_l{l}") + getattr(lstm, f"bias_hh_l{l}")).detach().to(dev) for l in range(L)]
    lin_w, lin_b = native.linear.weight.detach().to(dev), native.linear.bias.detach().to(dev)
    x = make_x(B, T, I).half()
    layers = [(w_ih[l].float().cpu().numpy(), w_hh[l].float().cpu().numpy(), fused[l].float().cpu().numpy(), None)
              for l in range(L)]
    lw, lb = lin_w.float().cpu().numpy(), lin_b.float().cpu().numpy()
    want = oracle.regressor_forward(x.float().numpy(), layers, lw, lb)
    want16 = oracle.regressor_forward(x.float().numpy(), layers, lw, lb, numerics="ref_fp16")
    return dict(x=x.to(dev), w_ih=w_ih, w_hh=w_hh, fused=fused, lin_w=lin_w, lin_b=lin_b, want=want,
                want16=want16)


def _args(s, fmt):
    out = []
    for l in range(4):
        if fmt == "torch":
            a, b = s["w_ih"][l], s["w_hh"][l]
        elif fmt == "packed":
            a, b = s["w_ih"][l].t().contiguous(), s["w_hh"][l].t().contiguous()
        elif fmt == "interleaved":
            a, b = kpairs(s["w_ih"][l]), kpairs(s["w_hh"][l])
        elif fmt == "projected":
            a, b = s["w_ih"][l], kpairs(s["w_hh"][l])
        out += [a, b, s["fused"][l]]
    return out + [s["lin_w"], s["lin_b"]]


def _check(got: torch.Tensor, s, rows=None, what=""):
    g = got.float().cpu().numpy()
    w, w16 = s["want"], s["want16"]
    if rows is not None:
        w, w16 = w[rows], w16[rows]
    mx, mn = assert_close(g, w, what=f"{what} vs fp32 oracle")
    mx16, mn16 = assert_close(g, w16, max_abs=REGRESSION_MAX_ABS, mean_abs=REGRESSION_MEAN_ABS,
                              what=f"{what} vs ref_fp16 oracle")
    _say(f"{what}: max_abs {mx:.2e} (fp32 oracle), {mx16:.2e} (ref_fp16 oracle)")


@pytest.mark.parametrize("name,fmt", [
    ("persistent_lstm4_forward", "torch"),
    ("persistent_lstm4_forward_packed", "packed"),
    ("persistent_lstm4_forward_interleaved", "interleaved"),
    ("persistent_lstm4_forward_monolithic", "interleaved"),
    ("persistent_lstm4_forward_projected", "projected"),
])
def test_four_layer_entry_points_match_oracle(setup, name, fmt):
    _say(f"entry point {name}")
    got = getattr(ext_mod, name)(setup["x"], *_args(setup, fmt))
    torch.cuda.synchronize()
    assert got.dtype == torch.float16 and tuple(got.shape) == (40, 24)
    _check(got, setup, what=name)


@pytest.mark.parametrize("name", ["persistent_lstm4_forward_projected_uniform",
                                  "persistent_lstm4_forward_projected_uniform_p4",
                                  "persistent_lstm4_forward_projected_uniform_p8"])
def test_uniform_entry_points_match_oracle(setup, name):
    """The reference dispatcher's uniform call: one row and a virtual batch size -> [1, O], then
    repeat_first_row; with more rows (or virtual_batch_size <= 0) every row is computed."""
    _say(f"entry point {name}")
    fn = getattr(ext_mod, name)
    args = _args(setup, "projected")
    one = fn(setup["x"].narrow(0, 0, 1), 4, *args)
    rep = ext_mod.repeat_first_row(one, 40)
    full = fn(setup["x"], 4, *args)
    none = fn(setup["x"].narrow(0, 0, 1), 0, *args)
    torch.cuda.synchronize()
    assert tuple(one.shape) == (1, 24) and tuple(rep.shape) == (40, 24) and tuple(full.shape) == (40, 24)
    assert torch.equal(rep, one.expand(40, -1))
    assert torch.equal(none, one)
    _check(one, setup, rows=[0], what=f"{name} one row")
    _check(full, setup, what=f"{name} all rows")


def test_generic_projected_entry_point_matches_oracle(setup):
    _say("entry point persistent_lstm_regressor_forward_generic_projected")
    got = ext_mod.persistent_lstm_regressor_forward_generic_projected(
        setup["x"], setup["w_ih"], setup["w_hh"], setup["fused"], setup["lin_w"], setup["lin_b"])
    torch.cuda.synchronize()
    _check(got, setup, what="generic_projected")


def test_entry_points_pack_once_per_weight_version(setup):
    """The reference dispatcher passes the same cached tensors each forward: the weights are packed
    once; an in-place update of one of them (a new version) repacks."""
    _say("entry point pack cache")
    lib = ext_mod._ext
    args = _args(setup, "projected")
    ext_mod.persistent_lstm4_forward_projected(setup["x"], *args)
    blob = lib._compat_blob
    ext_mod.persistent_lstm4_forward_projected(setup["x"], *args)
    assert lib._compat_blob is blob
    fused0 = args[2].clone()
    args[2].add_(0.5)
    try:
        got = ext_mod.persistent_lstm4_forward_projected(setup["x"], *args)
        assert lib._compat_blob is not blob
        torch.cuda.synchronize()
        d = (got.float() - torch.as_tensor(setup["want"], device="cuda")).abs().max().item()
        assert d > 1e-2, "a changed bias must change the output"
    finally:
        args[2].copy_(fused0)


def test_uniform_cache_survives_allocator_reuse():
    """A torch.ones input is detected as uniform; after it is freed, a random input of the same size
    allocated at the same address (factory tensors both have version 0) must be computed row by row.
    The reference's key (data_ptr, ..., _version; model.py:506-520) would reuse the cached True."""
    I, H, L, O, B, T = 5, 128, 2, 6, 64, 50
    _say("uniform cache vs allocator reuse")
    native = make_regressor(I, H, L, O)
    model = PersistentLSTMRegressor.from_native_module(native).to("cuda").half().eval()
    x1 = torch.ones(B, T, I, device="cuda", dtype=torch.float16)
    ptr = x1.data_ptr()
    out1 = model(x1)
    torch.cuda.synchronize()
    assert torch.equal(out1, out1[:1].expand_as(out1))
    del x1
    x2 = torch.randn(B, T, I, device="cuda", dtype=torch.float16, generator=torch.Generator("cuda").manual_seed(3))
    assert x2.data_ptr() == ptr and x2._version == 0, "the allocator did not reuse the block; test is void"
    out2 = model(x2)
    torch.cuda.synchronize()
    layers = [tuple(getattr(native.lstm, f"{n}_l{l}").detach().half().float().numpy()
                    for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")) for l in range(L)]
    want = oracle.regressor_forward(x2.float().cpu().numpy(), layers,
                                    native.linear.weight.detach().half().float().numpy(),
                                    native.linear.bias.detach().half().float().numpy())
    assert_close(out2.float().cpu().numpy(), want, what="reused-address random input")
    assert not torch.equal(out2, out2[:1].expand_as(out2))
