"""Converter interface types (mirrors torchtitan_npu/converters/model_custom_interface.py:15-60).

``ModelCustomConverter`` receives the torchtitan ``ModelSpec`` (anything with a ``name``)
and rewrites a built model in place; ``ModelCustomConfig`` bundles a converter with the
optional plan / state-dict updaters under a registered name.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Any


class ModelCustomConverter(ABC):
    def __init__(self, model_spec: Any):
        self.model_spec = model_spec
        self.model_name = getattr(model_spec, "name", None)

    @abstractmethod
    def convert(self, model) -> None:
        """Rewrite ``model`` in place."""


class ParallelizePlanUpdater(ABC):
    @classmethod
    @abstractmethod
    def update(cls, parallelize_plan):
        """Return the updated tensor-parallel plan."""


class StateDictUpdater(ABC):
    @classmethod
    @abstractmethod
    def to_hf(cls, state_dict: dict[str, Any]) -> dict[str, Any]:
        """Map a native state dict to the HF layout."""

    @classmethod
    @abstractmethod
    def from_hf(cls, state_dict: dict[str, Any]) -> dict[str, Any]:
        """Map an HF state dict to the native layout."""


@dataclass
class ModelCustomConfig:
    """A named model customisation: converter plus optional updaters."""

    name: str = "default"
    model_converter: type[ModelCustomConverter] | None = None
    parallelize_plan_updater: type[ParallelizePlanUpdater] | None = None
    state_dict_updater: type[StateDictUpdater] | None = None
