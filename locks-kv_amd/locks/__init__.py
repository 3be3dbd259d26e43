"""LOCKS decode hot path for AMD Instinct MI355X (gfx950).

Public API (same as the reference package, src/locks/__init__.py:23-31):
    from locks import LocksConfig, register

Layout:
    config.py            LocksConfig
    _lib.py              ctypes binding of liblocks_hip.so (HIP kernels)
    selection/           Rki4State, summary build, scorer, page selection
    attention/           split-K sparse paged decode + LSE merge
    backend/             plugin registration and the per-layer hot-path glue
"""
from __future__ import annotations

from .config import LocksConfig  # noqa: F401

__all__ = ["LocksConfig", "register"]

__version__ = "0.1.3+mi355x"


def register(overrides: dict | None = None) -> None:
    """Plugin entry point (vLLM ``general_plugins``); see backend.register."""
    from .backend.register import register as _register
    _register(overrides)
