"""The reference's import names resolve to this build (CPU: no kernel is launched).

The scripts the north star names import `from persistent_lstm_hip import convert_regressor_module`
(persistent_lstm_hip/LSTM-hip.py:7) and `from persistent_lstm_hip.model import
PersistentLSTMRegressor, StandardLSTMRegressor` (benchmark_persistent_lstm.py:5-8); the reference's
package loads its extension as `persistent_lstm_hip_ext` (extension.py:7-12), whose pybind module
exports ten functions (bindings.cpp:154-165).
"""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT_IMPORTS = """
from persistent_lstm_hip import convert_regressor_module
from persistent_lstm_hip.model import (
    PersistentLSTMRegressor,
    StandardLSTMRegressor,
)
from persistent_lstm_hip import (PersistentLSTM, PersistentLSTM4LayerRegressor, NativeModuleFallback,
                                 convert_lstm_module, replace_lstm_inplace, convert_model_copy)
from persistent_lstm_hip.api import convert_regressor_module as c2
from persistent_lstm_hip.packing import pack_lstm_module, pack_regressor_module, PackedLSTMWeights
from persistent_lstm_hip.extension import load_extension
import persistent_lstm_hip_amd
assert PersistentLSTMRegressor is persistent_lstm_hip_amd.PersistentLSTMRegressor
assert convert_regressor_module is c2 is persistent_lstm_hip_amd.convert_regressor_module
assert PersistentLSTM4LayerRegressor is PersistentLSTMRegressor
ext = load_extension()
assert ext is not None and ext is persistent_lstm_hip_amd.load_extension()
print("ok")
"""

REFERENCE_EXPORTS = [
    "persistent_lstm4_forward", "persistent_lstm4_forward_packed", "persistent_lstm4_forward_interleaved",
    "persistent_lstm4_forward_projected", "persistent_lstm4_forward_projected_uniform",
    "persistent_lstm4_forward_projected_uniform_p4", "persistent_lstm4_forward_projected_uniform_p8",
    "persistent_lstm4_forward_monolithic", "persistent_lstm_regressor_forward_generic_projected",
    "repeat_first_row",
]


def test_reference_script_imports_resolve_in_a_fresh_interpreter():
    env = dict(os.environ, PYTHONPATH=ROOT)
    out = subprocess.run([sys.executable, "-c", SCRIPT_IMPORTS], cwd="/tmp", env=env, capture_output=True, text=True)
    assert out.returncode == 0, out.stderr[-2000:]
    assert out.stdout.strip().endswith("ok")


def test_extension_module_exports_the_reference_entry_points():
    import persistent_lstm_hip_ext as ext_mod

    from persistent_lstm_hip_amd.extension import REFERENCE_ENTRY_POINTS, load_extension

    assert list(REFERENCE_ENTRY_POINTS) == REFERENCE_EXPORTS
    lib = load_extension()
    for name in REFERENCE_EXPORTS:
        fn = getattr(ext_mod, name)
        assert callable(fn)
        assert getattr(fn, "__func__", None) is getattr(type(lib), name), name
    assert sorted(ext_mod.__all__) == sorted(REFERENCE_EXPORTS)


def test_reference_loader_protocol_finds_the_module():
    """The reference loader is importlib.import_module("persistent_lstm_hip_ext") in a try block."""
    import importlib

    mod = importlib.import_module("persistent_lstm_hip_ext")
    assert hasattr(mod, "persistent_lstm4_forward_projected_uniform_p4")


@pytest.mark.parametrize("name", REFERENCE_EXPORTS[:8])
def test_four_layer_entry_points_check_their_argument_count(name):
    import persistent_lstm_hip_ext as ext_mod
    import torch

    fn = getattr(ext_mod, name)
    x = torch.zeros(1, 2, 5)
    args = (x, 4) if "uniform" in name else (x,)
    with pytest.raises(ValueError, match="12 per-layer tensors"):
        fn(*args, *([torch.zeros(1)] * 3))
