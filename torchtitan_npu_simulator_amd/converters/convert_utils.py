"""In-place patch helpers (reference: converters/convert_utils.py:159-180).

``replace_methods`` swaps ``class_name.method_name`` for ``new_method`` on every class of
that name found among the model's submodules and/or in the modules of ``package``;
it returns how many classes were patched.
"""

from __future__ import annotations

import sys
from typing import Callable


def _classes_named(class_name: str, model=None, package: str | None = None) -> list[type]:
    found: list[type] = []
    if model is not None:
        for m in model.modules():
            for cls in type(m).__mro__:
                if cls.__name__ == class_name and cls not in found:
                    found.append(cls)
    if package is not None:
        for mod_name, mod in list(sys.modules.items()):
            if mod is None or not (mod_name == package or mod_name.startswith(package + ".")):
                continue
            cls = getattr(mod, class_name, None)
            if isinstance(cls, type) and cls not in found:
                found.append(cls)
    return found


def replace_methods(class_name: str, method_name: str, new_method: Callable, model=None,
                    package: str | None = None) -> int:
    classes = _classes_named(class_name, model=model, package=package)
    for cls in classes:
        setattr(cls, method_name, new_method)
    return len(classes)


def replace_module_with_name(model, name: str, new) -> None:
    parent_name, _, attr = name.rpartition(".")
    parent = model.get_submodule(parent_name) if parent_name else model
    setattr(parent, attr, new)
