"""ctypes binding of liblocks_hip.so (the C ABI in include/locks_hip.h).

The product path has exactly one implementation: the HIP kernels in this
library.  If the library is missing the import of any hot-path entry raises
``LocksLibraryError`` -- there is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import os

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "liblocks_hip.so")
ABI_VERSION = 10

_c = ctypes
_i32, _i64, _f32, _f64, _p = _c.c_int32, _c.c_int64, _c.c_float, _c.c_double, _c.c_void_p



class TierSrc(_c.Structure):
    """locks_tier_src: the DRAM-tier V (and mem-kv K) source of the split decode."""
    _fields_ = [("hot_v", _p), ("stage_v", _p), ("pool_v", _p),
                ("hot_k", _p), ("stage_k", _p), ("pool_k", _p),
                ("page2slot", _p), ("vbo", _p),
                ("stage_stride_block", _i64), ("stage_stride_tok", _i64), ("stage_stride_head", _i64),
                ("num_blocks", _i32), ("hot_slots", _i32), ("stage_blocks", _i32), ("layer", _i32),
                ("k_tier", _i32), ("n_kv", _i32), ("page", _i32), ("head_dim", _i32),
                ("num_layers", _i32)]


# name -> (restype, argtypes); mirrors include/locks_hip.h one to one
SIGNATURES = {
    "locks_abi_version": (_i32, []),
    "locks_last_error": (_c.c_char_p, []),
    "locks_derive_params": (_i32, [_p, _i32, _i32, _i32, _i32, _i32, _f64, _p, _p, _p, _p]),
    "locks_score_auto_chunk": (_i32, [_i32, _i32, _i32]),
    "locks_score_num_chunks": (_i32, [_i32, _i32]),
    "locks_score_rki4": (_i32, [_p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _i32, _p, _i64, _i32,
                                _p, _p, _i32, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p]),
    "locks_select_workspace_bytes": (_i64, [_i32, _i32, _i32]),
    "locks_select_nrm_topb": (_i32, [_p, _p, _i32, _p, _p, _p, _p, _p, _p, _p, _i64,
                                     _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "locks_decode_splitk": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                                   _i32, _p, _i64, _i32, _p, _i64, _i64, _i32, _p, _i64, _p,
                                   _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                   _f32, _p]),
    "locks_decode_splitk_tier": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                                        _i32, _p, _i64, _i32, _p, _i64, _i64, _i32, _p, _i64, _p,
                                        _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                        _f32, _p, _p]),
    "locks_host_device_pointer": (_i32, [_p, _p]),
    "locks_tier_invalidate": (_i32, [_p, _i64, _i32, _p, _p, _i32, _p, _p, _p, _i32, _i32, _i32,
                                     _i32, _i32, _p]),
    "locks_tier_stage_begin": (_i32, [_p, _i64, _i32, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _i32,
                                      _p, _i32, _p, _i32, _i32, _i32, _p]),
    "locks_tier_flush_copy": (_i32, [_p, _p, _i32, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p,
                                     _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "locks_tier_scatter": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i32, _p, _p, _p, _i64, _i64,
                                  _i64, _i32, _i32, _i32, _i32, _i32, _p]),
    "locks_tier_plan": (_i32, [_p, _i64, _i64, _i32, _p, _i64, _p, _i64, _i32, _p, _i32, _p, _p,
                               _p, _p, _p, _p, _p, _p, _p, _i32, _p, _i32, _i32, _i32, _i32, _p]),
    "locks_tier_fetch": (_i32, [_p, _p, _i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p,
                                _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "locks_decode_fused": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                                  _i32, _p, _i64, _i32, _p, _i64, _i64, _i32, _p, _i64, _p,
                                  _p, _p, _p, _p, _p, _i64, _i64, _i32,
                                  _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p]),
    "locks_build_rki4": (_i32, [_p, _i64, _i64, _i64, _i32, _p, _i32, _i32, _i32, _i32,
                                _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "locks_refresh_blocks": (_i32, [_i32, _p, _i64, _p, _i32, _p, _i32, _i32, _i32, _i32, _p,
                                    _i32, _i64, _i64, _i64, _i32, _p, _i64, _p, _p, _p, _p]),
    "locks_build_rki4_layers": (_i32, [_p, _i32, _i64, _i64, _i64, _i32, _p, _p, _i32, _i32,
                                       _i32, _i32, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "locks_calib_read": (_i32, [_p, _i64, _p, _p]),
    "locks_pack_rki4": (_i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p]),
    "locks_mla_score": (_i32, [_p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p,
                               _i64, _i32, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _i32,
                               _i32, _f32, _p]),
    "locks_mla_score_auto_chunk": (_i32, [_i32, _i32]),
    "locks_mla_build_rope": (_i32, [_p, _i64, _i64, _i32, _p, _i32, _p, _p, _p, _p]),
    "locks_mla_decode_splitk": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i32, _p, _i64, _i32, _p,
                                       _i64, _i32, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32,
                                       _i32, _i32, _i32, _f32, _p]),
    "locks_mla_decode_merge": (_i32, [_p, _p, _p, _p, _i32, _p, _i64, _i64, _i32, _p, _i64, _i32,
                                      _i32, _i32, _i32, _i32, _p]),
    "locks_mla_decode_dense": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i32, _p, _i64, _i32, _p,
                                      _p, _p, _p, _p, _i64, _i64, _i32, _p, _i64, _i32, _i32,
                                      _i32, _i32, _i32, _i32, _f32, _p]),
    "locks_decode_fused_noalloc": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64,
                                          _i64, _i32, _p, _i64, _i32, _p, _i64, _i64, _i32, _p,
                                          _i64, _p, _p, _i64, _i64, _i32, _i32, _i32, _i32, _i32,
                                          _i32, _i32, _i32, _i32, _f32, _p]),
    "locks_decode_dense": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                                  _i32, _p, _i64, _i32, _p, _p, _p, _p, _p, _i64, _i64, _i32,
                                  _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p]),
    "locks_decode_merge": (_i32, [_p, _p, _p, _p, _i64, _i32, _p, _i64, _i64, _i32, _i32, _i32,
                                  _i32, _i32, _i32, _i32, _i32, _p]),
}


class LocksLibraryError(RuntimeError):
    """liblocks_hip.so is missing, stale or rejected a call."""


_LIB = None


def lib_path() -> str:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and type the HIP library; raise if it is absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.isfile(_LIB_PATH):
        raise LocksLibraryError(
            f"{_LIB_PATH} not found: build it with `python locks-kv_amd/build_lib.py` "
            "(or __graft_entry__.build()). The LOCKS hot path has no fallback.")
    lib = ctypes.CDLL(_LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    v = lib.locks_abi_version()
    if v != ABI_VERSION:
        raise LocksLibraryError(f"liblocks_hip ABI {v} != expected {ABI_VERSION}; rebuild it")
    _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().locks_last_error().decode(errors="replace")
        raise RuntimeError(f"locks: {what} failed ({rc}): {msg}")


def ptr(t) -> int:
    """Device pointer of a torch tensor (None -> NULL)."""
    return 0 if t is None else int(t.data_ptr())


def rows_arg(st) -> int:
    """slab_row_bytes argument for a summary state: the address of its six
    row strides (a state with packed rows), or NULL (contiguous slabs)."""
    rb = getattr(st, "slab_row_bytes", None)
    return 0 if rb is None else _c.addressof(rb)


def stream_ptr(device=None) -> int:
    import torch
    return int(torch.cuda.current_stream(device).cuda_stream)
