"""Qwen3 decode engine bindings (include/xpu_qwen3.h)."""
from __future__ import annotations

from . import library


def available() -> bool:
    return hasattr(library(), "xpu_qwen3_create")
