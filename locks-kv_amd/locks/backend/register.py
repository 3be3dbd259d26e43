"""Plugin registration (vLLM ``general_plugins`` entry point).

Mirrors src/locks/backend/register.py:123-183: inert unless ``LOCKS_CONFIG``
is set or overrides are given, disabled by ``LOCKS_DISABLE``; otherwise the
config is loaded once and the attention-backend selector is patched so the
FlashAttention backend resolves to the LOCKS backend.  On ROCm the selector
lives on ``vllm.platforms.rocm.RocmPlatform`` (the reference patches the CUDA
platform only).  When vLLM is not installed (as in this image) registration
stops after loading the config: the hot path is then driven directly
through ``backend.engine.LocksEngine`` / ``backend._runtime``.  When vLLM-ROCm
is importable but the vLLM backend class is not shipped (this build),
registration refuses with ``NotImplementedError`` instead of patching the
selector to a missing class.
"""
from __future__ import annotations

import os

from ..config import LocksConfig
from . import _runtime

_APPLIED = False
_OUR_PATH = "locks.backend.attn.LocksAttentionBackend"


def register(overrides: dict | None = None) -> None:
    global _APPLIED
    if _APPLIED or os.environ.get("LOCKS_DISABLE"):
        return
    if overrides is None and not os.environ.get("LOCKS_CONFIG"):
        print("[locks] register: no LOCKS_CONFIG and no overrides -> plugin INERT.",
              flush=True)
        return
    cfg = LocksConfig.load(overrides)
    _runtime.set_config(cfg)
    try:
        from vllm.platforms import rocm  # noqa: F401
    except Exception:  # vLLM absent: config registered, no selector to patch
        _APPLIED = True
        print(f"[locks] registered config (variant={cfg.variant}); vLLM not importable, "
              "backend selector not patched", flush=True)
        return
    import importlib.util
    if importlib.util.find_spec(_OUR_PATH.rsplit(".", 1)[0]) is None:
        # the vLLM attention-backend class is not shipped by this build:
        # refuse here rather than let vLLM fail later on a missing import
        raise NotImplementedError(
            "locks: vLLM-ROCm is importable but this build ships no vLLM attention backend "
            f"class ({_OUR_PATH}); drive the decode path with locks.backend.engine.LocksEngine")
    target = next(k for k in rocm.RocmPlatform.__mro__ if "get_attn_backend_cls" in k.__dict__)
    orig = target.__dict__["get_attn_backend_cls"].__func__

    def get_attn_backend_cls(cls, *args, **kwargs):
        path = orig(cls, *args, **kwargs)
        if isinstance(path, str) and path.endswith("FlashAttentionBackend"):
            return _OUR_PATH
        return path

    target.get_attn_backend_cls = classmethod(get_attn_backend_cls)
    _APPLIED = True
    print("[locks] registered (patched RocmPlatform.get_attn_backend_cls)", flush=True)
