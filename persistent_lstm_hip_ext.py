"""The reference's compiled extension module name, `persistent_lstm_hip_ext`, for this build.

The reference's own Python package loads its extension with
`importlib.import_module("persistent_lstm_hip_ext")` (persistent_lstm_hip/extension.py:7-12) and
calls the ten functions its pybind module exports (bindings.cpp:154-165).  This module exports the
same ten names, bound to the MI355X library through persistent_lstm_hip_amd.extension, so that
package can run on this build with only its extension swapped.  Like a missing compiled extension,
importing it raises ImportError when the native library cannot be loaded (the reference's loader
then returns None).  Inputs must be HIP tensors: there is no CPU branch (the reference's
persistent_lstm_op.cpp falls back to its ATen CPU path; this build raises ValueError instead).
"""
from persistent_lstm_hip_amd.extension import REFERENCE_ENTRY_POINTS, load_error, load_extension

_ext = load_extension()
if _ext is None:
    raise ImportError(f"persistent_lstm_hip_ext: native library unavailable: {load_error()}")

persistent_lstm4_forward = _ext.persistent_lstm4_forward
persistent_lstm4_forward_packed = _ext.persistent_lstm4_forward_packed
persistent_lstm4_forward_interleaved = _ext.persistent_lstm4_forward_interleaved
persistent_lstm4_forward_projected = _ext.persistent_lstm4_forward_projected
persistent_lstm4_forward_projected_uniform = _ext.persistent_lstm4_forward_projected_uniform
persistent_lstm4_forward_projected_uniform_p4 = _ext.persistent_lstm4_forward_projected_uniform_p4
persistent_lstm4_forward_projected_uniform_p8 = _ext.persistent_lstm4_forward_projected_uniform_p8
persistent_lstm4_forward_monolithic = _ext.persistent_lstm4_forward_monolithic
persistent_lstm_regressor_forward_generic_projected = _ext.persistent_lstm_regressor_forward_generic_projected
repeat_first_row = _ext.repeat_first_row

__all__ = list(REFERENCE_ENTRY_POINTS)
