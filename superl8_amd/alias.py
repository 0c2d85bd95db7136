"""Serve this package under the reference's module names.

``install()`` registers ``superl8``, ``superl8.ops``, ``superl8._C``,
``superl8.quant`` (with ``.core``, ``.rotation`` and ``.lloydmax``),
``superl8.format`` and ``superl8.gguf`` in ``sys.modules``
so that code written against the reference's hot-path surface
(``from superl8.ops import attn_int8_fwd``, ``from superl8 import _C``, ...)
runs on this build unchanged. Names that already exist in ``sys.modules`` (the
reference package itself, if it is importable) are left alone unless
``force=True``.
"""
from __future__ import annotations

import sys

_SUBMODULES = ("ops", "_C", "quant", "quant.core", "quant.rotation", "quant.lloydmax", "format", "gguf")


def install(force: bool = False) -> None:
    import importlib

    pkg = importlib.import_module("superl8_amd")
    if force or "superl8" not in sys.modules:
        sys.modules["superl8"] = pkg
    for name in _SUBMODULES:
        key = f"superl8.{name}"
        if force or key not in sys.modules:
            sys.modules[key] = importlib.import_module(f"superl8_amd.{name}")


def uninstall() -> None:
    """Remove the names install() registered (only those that point at this package)."""
    for key in ["superl8"] + [f"superl8.{n}" for n in _SUBMODULES]:
        mod = sys.modules.get(key)
        if mod is not None and getattr(mod, "__name__", "").startswith("superl8_amd"):
            del sys.modules[key]
