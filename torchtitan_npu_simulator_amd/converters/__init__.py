"""ModelConverter plugin API of the DSA path: ``register_model_converter``,
``get_model_converter_config("npu_dsa" | "npu_smla")`` and the converters themselves.
Importing this package registers both converters (the reference's
converters/__init__.py:30-48 does the same by auto-import)."""

from .model_custom_interface import ModelCustomConfig, ModelCustomConverter  # noqa: F401
from .registry import (  # noqa: F401
    ModelCustomConfigConverter,
    get_model_converter_config,
    has_npu_converter,
    register_model_converter,
    registry,
    set_model_spec,
)
from . import dsa, npu_smla  # noqa: F401,E402  (registers "npu_dsa" and "npu_smla")
