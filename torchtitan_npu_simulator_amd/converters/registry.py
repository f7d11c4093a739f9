"""Model-converter registry (the reference's plugin API, converters/registry.py:11-40 and
converters/framework/model_custom_config_registry.py:11-80).

``@register_model_converter("npu_dsa")`` on a ``ModelCustomConfig`` subclass creates a
torchtitan model-converter class named ``npu_dsaModelCustomConfigConverter`` whose
``Config`` (``get_model_converter_config("npu_dsa")``) is what a trainer recipe lists in
``model_converters``.  When torchtitan is importable the generated classes derive from
``torchtitan.config.Configurable`` / ``torchtitan.protocols.model_converter.ModelConverter``
exactly as the reference's do; otherwise they derive from the small stand-ins below so
the converters stay usable (and testable) without torchtitan.
"""

from __future__ import annotations

import logging
from typing import Any

from .model_custom_interface import ModelCustomConfig

logger = logging.getLogger(__name__)

try:  # torchtitan present: the generated classes plug into its converter protocol
    from torchtitan.config import Configurable as _Configurable  # type: ignore
    from torchtitan.protocols.model_converter import ModelConverter as _ModelConverter  # type: ignore

    _ConfigBase = _Configurable.Config
    _ConverterBases: tuple = (_Configurable, _ModelConverter)
except Exception:  # pragma: no cover - exercised in this repository's tests

    class _ConfigBase:  # minimal Configurable.Config stand-in
        def build(self, **kwargs):
            return self._owner(self, **kwargs)

    _ConverterBases = ()

_MODEL_SPEC: Any = None


def set_model_spec(model_spec: Any) -> None:
    """Model spec handed to converters built without an explicit ``model_spec`` (the
    reference reads it from its trainer-config stash)."""
    global _MODEL_SPEC
    _MODEL_SPEC = model_spec


class ModelCustomConfigConverter(*_ConverterBases):
    """Applies a ``ModelCustomConfig`` (reference: framework/model_custom_config_converter.py:26-66)."""

    _model_config: ModelCustomConfig

    def __init__(self, config=None, *, parallel_dims=None, model_compile_enabled: bool = False, model_spec=None):
        self.config = config
        self.parallel_dims = parallel_dims
        self.model_compile_enabled = model_compile_enabled
        self.model_spec = model_spec if model_spec is not None else _MODEL_SPEC
        self.model_name = getattr(self.model_spec, "name", None)

    def convert(self, model) -> None:
        name = self._model_config.name
        try:
            logger.info(f"[ModelCustomConfigConverter] Applied {name!r} start ...")
            conv = self._model_config.model_converter
            if conv is not None:
                conv(self.model_spec).convert(model)
                logger.info(f"[ModelCustomConfigConverter] Applied {conv}.")
            for attr in ("parallelize_plan_updater", "state_dict_updater"):
                if getattr(self._model_config, attr) is not None:
                    logger.info(f"[ModelCustomConfigConverter] {attr} is not used by the DSA path; skipped.")
            logger.info(f"[ModelCustomConfigConverter] Applied {name!r} end.")
        except Exception as e:
            raise RuntimeError(f"Failed to apply custom model config {name!r} : {e}") from e

    def post_optimizer_hook(self, model) -> None:  # torchtitan ModelConverter protocol
        return None


class _ConverterRegistry:
    _instance = None

    def __new__(cls):
        if cls._instance is None:
            inst = super().__new__(cls)
            inst._model_configs = {}
            inst._converter_classes = {}
            cls._instance = inst
        return cls._instance

    def register(self, name: str):
        def decorator(config):
            config.name = name
            self._model_configs[name] = config
            self._register_as_model_converter(name, config)
            return config

        return decorator

    def get_config(self, name: str):
        cls = self._converter_classes.get(name)
        return None if cls is None else cls.Config()

    def get(self, name: str):
        return self._model_configs.get(name)

    def converter_class(self, name: str):
        return self._converter_classes.get(name)

    def _register_as_model_converter(self, name: str, config) -> None:
        converter_cls = type(f"{name}ModelCustomConfigConverter", (ModelCustomConfigConverter,), {"_model_config": config})

        def to_dict(self):
            return {"name": self.name}

        config_cls = type(f"{converter_cls.__name__}Config", (_ConfigBase,),
                          {"name": name, "to_dict": to_dict, "__annotations__": {}})
        config_cls._owner = converter_cls
        converter_cls.Config = config_cls
        self._converter_classes[name] = converter_cls


_registry = _ConverterRegistry()


def registry() -> _ConverterRegistry:
    return _registry


def register_model_converter(name: str):
    return _registry.register(name)


def get_model_converter_config(name: str):
    return _registry.get_config(name)


def has_npu_converter(converters: list, name: str) -> bool:
    """True if ``converters`` holds a Config (or converter class) registered under ``name``."""
    for c in converters:
        owner = getattr(c, "_owner", None) or c
        model_config = getattr(owner, "_model_config", None)
        if model_config is not None and getattr(model_config, "name", None) == name:
            return True
    return False
