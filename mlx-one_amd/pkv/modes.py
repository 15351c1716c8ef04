"""Capability errors, as in the reference (src/mlx_one/engine/modes.py:16-17)."""


class ModelCapabilityUnsupported(ValueError):
    code = "MODEL_CAPABILITY_UNSUPPORTED"
