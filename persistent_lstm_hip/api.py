"""`persistent_lstm_hip.api` (reference api.py:10-43) -> persistent_lstm_hip_amd.api."""
from persistent_lstm_hip_amd.api import (  # noqa: F401
    convert_lstm_module,
    convert_model_copy,
    convert_regressor_module,
    replace_lstm_inplace,
)
