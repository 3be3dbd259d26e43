"""LocksConfig: the single configuration object of the LOCKS plugin.

Field names, defaults, validation and the ``load()`` precedence mirror the
reference (src/locks/config.py:26-214) so an existing ``LOCKS_CONFIG`` file
works unchanged.  Every variant is served: ``fast`` (K+V resident) and the
DRAM-tier ``mem-v`` / ``mem-kv`` (V, or K and V, decoded from the tier of
``locks.tier``); ``mem_summary_cache`` (summary records in the engine page)
is refused when state is created.
"""
from __future__ import annotations

import dataclasses
import json
import os
from typing import Literal, Optional

Variant = Literal["fast", "mem-v", "mem-kv"]
Table = Literal["kv-union", "q-head", "kv-shared"]


@dataclasses.dataclass(frozen=True)
class LocksConfig:
    variant: Variant = "fast"
    coverage: float = 0.95
    budget: Optional[float] = None
    budget_pages: Optional[int] = None
    table: Table = "kv-union"
    sink_pages: int = 1
    window_pages: int = 1
    r8_screen: bool = False
    r8_rank: int = 8
    quad_combine: Literal["max", "nrm"] = "nrm"
    rki4_zsplit: Optional[int] = None
    hot_slots: int = 0
    hot_ratio: float = 6.0
    v_blocks: Optional[int] = None
    max_pool_gb: float = 256.0
    mem_k_only: bool = True
    mem_summary_cache: bool = False
    use_cuda: bool = True
    force_eager: bool = False

    @property
    def is_mem(self) -> bool:
        return self.variant in ("mem-v", "mem-kv")

    @property
    def offload_k(self) -> bool:
        return self.variant == "mem-kv"

    def __post_init__(self) -> None:
        if self.variant not in ("fast", "mem-v", "mem-kv"):
            raise ValueError(f"unknown variant {self.variant!r}")
        if self.offload_k and not self.r8_screen:
            object.__setattr__(self, "r8_screen", True)
        if not (0.0 < self.coverage <= 1.0):
            raise ValueError(f"coverage must be in (0,1], got {self.coverage}")
        if self.budget is not None and not (0.0 < self.budget <= 1.0):
            raise ValueError(f"budget must be in (0,1], got {self.budget}")
        if self.rki4_zsplit is not None and not (1 <= self.rki4_zsplit <= 65535):
            raise ValueError(
                f"rki4_zsplit must be None (auto) or in [1, 65535], got {self.rki4_zsplit}")
        if self.quad_combine not in ("max", "nrm"):
            raise ValueError(f"quad_combine must be 'max' or 'nrm', got {self.quad_combine!r}")
        if not (0.0 < float(self.hot_ratio) <= 64.0):
            raise ValueError(f"hot_ratio must be in (0, 64], got {self.hot_ratio}")
        if self.sink_pages < 0:
            raise ValueError(f"sink_pages must be >= 0, got {self.sink_pages}")
        if self.window_pages < 1:
            raise ValueError(f"window_pages must be >= 1, got {self.window_pages}")
        if self.mem_summary_cache:
            if self.variant != "mem-kv":
                raise ValueError("mem_summary_cache requires variant='mem-kv' (K must live "
                                 f"in the tier); got {self.variant!r}")
            if not self.mem_k_only:
                raise ValueError("mem_summary_cache requires mem_k_only=True")

    @classmethod
    def load(cls, overrides: Optional[dict] = None) -> "LocksConfig":
        """``LOCKS_CONFIG`` (file path, .json/.yaml, or inline JSON) updated
        by ``overrides``; then the LOCKS_MEM_SUMMARY_CACHE / LOCKS_RKI4_Z env
        escapes when the key is not set explicitly.  Unknown keys raise."""
        data: dict = {}
        spec = os.environ.get("LOCKS_CONFIG")
        if spec:
            if os.path.isfile(spec):
                with open(spec) as fh:
                    text = fh.read()
                if spec.endswith((".yaml", ".yml")):
                    import yaml
                    data = yaml.safe_load(text) or {}
                else:
                    data = json.loads(text)
            else:
                data = json.loads(spec)
        if overrides:
            data.update({k: v for k, v in overrides.items() if v is not None})
        sc = os.environ.get("LOCKS_MEM_SUMMARY_CACHE")
        if sc is not None and "mem_summary_cache" not in data:
            data["mem_summary_cache"] = sc not in ("", "0", "false", "False")
        z = os.environ.get("LOCKS_RKI4_Z")
        if z is not None and "rki4_zsplit" not in data:
            data["rki4_zsplit"] = int(z)
        unknown = set(data) - {f.name for f in dataclasses.fields(cls)}
        if unknown:
            raise ValueError(f"unknown LocksConfig keys: {sorted(unknown)}")
        return cls(**data)
