"""The roofline arithmetic of bench.py, on the CPU: its algorithmic FLOP count per forward against a
count derived independently from the shapes of an nn.LSTM + nn.Linear's parameters (each weight
matrix [rows, cols] applied once per row of the batch and step costs 2 * rows * cols FLOPs), and the
C2 figure the committed profiles and the bench line quote."""
from __future__ import annotations

import importlib.util
import os

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _flops_from_parameters(I, H, L, O, B, T) -> float:
    """Dense-contraction FLOPs of one forward, from the parameter shapes: the recurrence applies
    weight_ih_l{k} and weight_hh_l{k} to every (row, step); the head applies the Linear weight to the
    last step's h of every row.  Biases and the cell's elementwise work are not contractions."""
    lstm = torch.nn.LSTM(I, H, num_layers=L, batch_first=True)
    head = torch.nn.Linear(H, O)
    per_row_step = 0
    for name, p in lstm.named_parameters():
        if name.startswith("weight_"):
            rows, cols = p.shape
            per_row_step += 2 * rows * cols
    per_row = 2 * head.weight.shape[0] * head.weight.shape[1]
    return float(B * T * per_row_step + B * per_row)


@pytest.mark.parametrize("geom", [(5, 128, 4, 24, 512, 1000), (5, 256, 4, 24, 512, 1000),
                                  (5, 512, 4, 24, 512, 1000), (7, 33, 1, 1, 3, 11), (40, 64, 3, 5, 9, 2)])
def test_algorithmic_flops_match_the_parameter_count(geom):
    bench = _bench()
    assert bench.algorithmic_flops(*geom) == _flops_from_parameters(*geom)


def test_c2_figure_quoted_by_the_profiles():
    # 4H (I + H) + 3 * 4H * 2H = 512 * 133 + 3 * 512 * 256 = 461,184 multiply-adds per (row, step),
    # x 2 x 512 x 1000, plus the head's 2 x 512 x 128 x 24
    bench = _bench()
    assert bench.algorithmic_flops(5, 128, 4, 24, 512, 1000) == 472386633728.0
    assert (bench.I, bench.H, bench.L, bench.O, bench.B, bench.T) == (5, 128, 4, 24, 512, 1000)
