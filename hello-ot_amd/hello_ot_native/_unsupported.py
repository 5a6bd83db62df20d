"""Module-level ``__getattr__`` for reference native functions without an MI355X counterpart."""
from __future__ import annotations


def missing(module: str, replacements: dict[str, str]):
    def __getattr__(name: str):
        if name.startswith("__"):
            raise AttributeError(name)
        hint = replacements.get(name)
        detail = f"; use {hint}" if hint else ""
        raise NotImplementedError(
            f"hello_ot_native.{module}.{name} is a tile-level reference kernel that the MI355X library fuses away"
            f"{detail}")
    return __getattr__
