"""ctypes front end of the CPU oracle (oracle/lstm_oracle.c) and of the reference's own CPU path
built into oracle/_ref/ (oracle/ref_driver.cpp around persistent_lstm_reference.cpp:42-64).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the checker.  The product package never imports this module.

Numerics modes (see the header of lstm_oracle.c for the reference file:line of each rule):
  "fp32"          -- textbook fp32 LSTM (what torch's CPU nn.LSTM computes), double accumulation
  "ref_fp16"      -- the reference kernels' storage: fp16-rounded fused bias, fp16 h every step,
                     fp32 c, fp16 head output.  Inputs/weights are rounded to fp16 by this wrapper.
  "ref_fp16_proj" -- as ref_fp16, with each step's input projection W_ih x rounded to fp16 before
                     the bias and recurrent terms are added (the reference's generic path, whose
                     projection is an fp16 torch::matmul).
  "ref_fp16_proj_l1" -- as ref_fp16_proj for layers >= 1, layer 0's projection unrounded (this
                     build's layer-sequential path with input_size <= 32, which projects layer 0
                     inside its recurrent kernel in fp32 and the other layers with its fp16 GEMM).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_ORACLE_SO = os.path.join(_HERE, "liblstm_oracle.so")
_REF_SO = os.path.join(_HERE, "_ref", "libref_lstm.so")
_REF_CPP = "/root/reference/persistent_lstm_hip/csrc/persistent_lstm_reference.cpp"

_lib = None
_ref = None

MUTATIONS = {
    "none": 0,
    "swap_if": 1,
    "drop_recurrent": 2,
    "transpose_whh": 3,
    "drop_bias_hh": 4,
    "no_tanh_c": 5,
    "gate_order_igfo": 6,
}

_F = ctypes.POINTER(ctypes.c_float)
_I32 = ctypes.POINTER(ctypes.c_int32)
_PF = ctypes.POINTER(_F)


def build(force: bool = False) -> None:
    """Compile the oracle (gcc) and, if the reference checkout is present, oracle/_ref."""
    if force or not os.path.exists(_ORACLE_SO):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liblstm_oracle.so"], check=True)
    if os.path.exists(_REF_CPP) and (force or not os.path.exists(_REF_SO)):
        subprocess.run(["make", "-C", _HERE, "ref"] + (["-B"] if force else []), check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_ORACLE_SO):
            build()
        lib = ctypes.CDLL(_ORACLE_SO)
        lib.oracle_lstm_forward.restype = ctypes.c_int
        lib.oracle_lstm_forward.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _F,
            _PF, _PF, _PF, _PF, _I32, _F, _F, ctypes.c_int, _I32, ctypes.c_int, _F, _F,
            _F, _F, _F, ctypes.c_int, ctypes.c_int,
        ]
        lib.oracle_linear.restype = ctypes.c_int
        lib.oracle_linear.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _F, _F, _F, _F, ctypes.c_int]
        lib.oracle_float_to_half_bits.restype = ctypes.c_uint16
        lib.oracle_float_to_half_bits.argtypes = [ctypes.c_float]
        lib.oracle_round_half_array.restype = None
        lib.oracle_round_half_array.argtypes = [_F, ctypes.c_int64]
        lib.oracle_max_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    return a.ctypes.data_as(_F)


def round_half(a) -> np.ndarray:
    """Round float32 values to the nearest fp16 (RNE) with the oracle's own converter."""
    out = _f32(a).copy()
    _load().oracle_round_half_array(_ptr(out), out.size)
    return out


def half_bits(value: float) -> int:
    return int(_load().oracle_float_to_half_bits(float(value)))


def max_threads() -> int:
    return int(_load().oracle_max_threads())


LayerWeights = Tuple[np.ndarray, np.ndarray, Optional[np.ndarray], Optional[np.ndarray]]


def lstm_forward(
    x,
    layers: Sequence[LayerWeights],
    *,
    lengths=None,
    h0=None,
    c0=None,
    numerics: str = "fp32",
    probe_steps: Sequence[int] = (),
    want_seq: bool = False,
    mutation: str = "none",
    threads: int = 0,
) -> Dict[str, np.ndarray]:
    """Stacked LSTM forward on the CPU.  x: [B,T,I]; layers: (w_ih [4H,K], w_hh [4H,H], b_ih, b_hh).

    Returns dict with h_n, c_n [L,B,H]; out_seq [B,T,H] if want_seq; probe_h/probe_c
    [P,L,B,H] for probe_steps.
    """
    lib = _load()
    mode = {"fp32": 0, "ref_fp16": 1, "ref_fp16_proj": 2, "ref_fp16_proj_l1": 3}[numerics]
    x = _f32(x)
    if x.ndim != 3:
        raise ValueError("x must be [B, T, I]")
    B, T, I = x.shape
    L = len(layers)
    H = int(np.asarray(layers[0][1]).shape[1])
    conv = round_half if mode else _f32
    if mode:
        x = round_half(x)
    keep: List[np.ndarray] = []
    wi, wh, bi, bh = (_F * L)(), (_F * L)(), (_F * L)(), (_F * L)()
    for l, (w_ih, w_hh, b_ih, b_hh) in enumerate(layers):
        a = conv(w_ih)
        b = conv(w_hh)
        if a.shape != (4 * H, I if l == 0 else H) or b.shape != (4 * H, H):
            raise ValueError(f"layer {l}: bad weight shapes {a.shape} {b.shape}")
        c = conv(b_ih) if b_ih is not None else np.zeros(4 * H, np.float32)
        d = conv(b_hh) if b_hh is not None else None
        keep += [a, b, c] + ([d] if d is not None else [])
        wi[l], wh[l], bi[l] = _ptr(a), _ptr(b), _ptr(c)
        bh[l] = _ptr(d) if d is not None else _F()
    lens = None
    if lengths is not None:
        lens = np.ascontiguousarray(np.asarray(lengths, dtype=np.int32))
        if lens.shape != (B,):
            raise ValueError("lengths must be [B]")
    h0a = conv(h0) if h0 is not None else None
    c0a = _f32(c0) if c0 is not None else None
    probes = np.ascontiguousarray(np.asarray(list(probe_steps), dtype=np.int32))
    P = probes.size
    probe_h = np.zeros((P, L, B, H), np.float32)
    probe_c = np.zeros((P, L, B, H), np.float32)
    out_seq = np.zeros((B, T, H), np.float32) if want_seq else None
    h_n = np.zeros((L, B, H), np.float32)
    c_n = np.zeros((L, B, H), np.float32)
    rc = lib.oracle_lstm_forward(
        B, T, I, H, L, _ptr(x), wi, wh, bi, bh,
        lens.ctypes.data_as(_I32) if lens is not None else None,
        _ptr(h0a), _ptr(c0a), mode,
        probes.ctypes.data_as(_I32) if P else None, P,
        _ptr(probe_h) if P else None, _ptr(probe_c) if P else None,
        _ptr(out_seq), _ptr(h_n), _ptr(c_n), MUTATIONS[mutation], int(threads),
    )
    if rc != 0:
        raise ValueError("oracle_lstm_forward rejected its arguments")
    res = {"h_n": h_n, "c_n": c_n}
    if want_seq:
        res["out_seq"] = out_seq
    if P:
        res["probe_h"], res["probe_c"] = probe_h, probe_c
    return res


def linear(inp, w, b, numerics: str = "fp32") -> np.ndarray:
    """bias + inp w^T (double accumulation); "ref_fp16": operands rounded to fp16 and the result
    rounded to fp16 as the reference's head kernel does (persistent_lstm_hip.cu:1662-1682)."""
    lib = _load()
    mode = {"fp32": 0, "ref_fp16": 1, "ref_fp16_proj": 1, "ref_fp16_proj_l1": 1}[numerics]
    conv = round_half if mode == 1 else _f32
    inp, w = conv(inp), conv(w)
    b = conv(b) if b is not None else None
    B, K = inp.shape
    O = w.shape[0]
    out = np.zeros((B, O), np.float32)
    if lib.oracle_linear(B, K, O, _ptr(inp), _ptr(w), _ptr(b), _ptr(out), mode) != 0:
        raise ValueError("oracle_linear rejected its arguments")
    return out


def regressor_forward(x, layers, linear_w, linear_b, *, lengths=None, numerics: str = "fp32",
                      mutation: str = "none", threads: int = 0) -> np.ndarray:
    """Linear(LSTM(x)[:, -1]) (reference.py:66-72).  With lengths, the head reads each row's state
    at its true last step, h_n[-1] (packed-sequence semantics)."""
    r = lstm_forward(x, layers, lengths=lengths, numerics=numerics, mutation=mutation, threads=threads)
    return linear(r["h_n"][-1], linear_w, linear_b, numerics=numerics)


# ---- the reference's own ATen CPU path, compiled from its sources into oracle/_ref ----

def ref_available() -> bool:
    return os.path.exists(_REF_SO)


def _load_ref():
    global _ref
    if _ref is None:
        import torch  # noqa: F401  (loads the libtorch the reference path links against)
        lib = ctypes.CDLL(_REF_SO)
        lib.ref_lstm4_forward.restype = ctypes.c_int
        lib.ref_lstm4_forward.argtypes = [ctypes.c_int] * 5 + [_F, _PF, _PF, _PF, _F, _F, _F, ctypes.c_int]
        lib.ref_num_threads.restype = ctypes.c_int
        _ref = lib
    return _ref


def ref_regressor_forward(x, layers, linear_w, linear_b, threads: int = 0) -> np.ndarray:
    """Run persistent_lstm4_forward_reference (reference.cpp:42-64) on float32 inputs.  It is
    fixed at 4 layers; the bias it takes is the fused b_ih + b_hh."""
    lib = _load_ref()
    x = _f32(x)
    B, T, I = x.shape
    if len(layers) != 4:
        raise ValueError("the reference CPU path is fixed at 4 layers")
    H = int(np.asarray(layers[0][1]).shape[1])
    keep = []
    wi, wh, bb = (_F * 4)(), (_F * 4)(), (_F * 4)()
    for l, (w_ih, w_hh, b_ih, b_hh) in enumerate(layers):
        a, b = _f32(w_ih), _f32(w_hh)
        c = _f32(b_ih) + (_f32(b_hh) if b_hh is not None else 0.0)
        c = _f32(c)
        keep += [a, b, c]
        wi[l], wh[l], bb[l] = _ptr(a), _ptr(b), _ptr(c)
    wl, bl = _f32(linear_w), _f32(linear_b)
    O = wl.shape[0]
    out = np.zeros((B, O), np.float32)
    if lib.ref_lstm4_forward(B, T, I, H, O, _ptr(x), wi, wh, bb, _ptr(wl), _ptr(bl), _ptr(out), int(threads)) != 0:
        raise RuntimeError("reference CPU path failed")
    return out


def ref_num_threads() -> int:
    return int(_load_ref().ref_num_threads())
