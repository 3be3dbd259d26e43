"""Per-layer hot-path glue: the select adapter and the decode dispatch.

Signatures follow the reference's runtime (src/locks/backend/_runtime.py:661
_rki4_select_adapter, :807 decode_dispatch, :841 resolve_selection), so an
attention impl written against them (backend/attn.py:371-378) is unchanged.
There is one implementation per stage -- the gfx950 HIP kernels -- and no
fallback: a missing library raises.
"""
from __future__ import annotations

from .. import _lib
from ..attention.decode import sparse_paged_decode_batched
from ..selection import Rki4State, derive_page_params
from ..selection.ops import rki4_score_state

_CFG = None


def set_config(cfg) -> None:
    global _CFG
    _CFG = cfg


def get_config():
    return _CFG


def _layer_index(st, kv_cache) -> int:
    layer_of = getattr(st, "_layer_of", None)
    if layer_of is None:
        raise RuntimeError("locks: Rki4State has no kv_cache -> layer map (_layer_of)")
    return layer_of[kv_cache.data_ptr()]


def _rki4_select_adapter(q, kv_cache, block_table, seq_lens, st, n_req, scale, cfg) -> None:
    """Stage A for one layer: score every selectable page from the summary
    slabs, combine the GQA group and write st.page_table / st.page_cnt.
    st.n_sel_hi etc. were derived by the builder for this step."""
    lidx = _layer_index(st, kv_cache)
    rki4_score_state(st, lidx, q, block_table, seq_lens, n_req, scale)


def decode_dispatch(q, kv_cache, block_table, seq_lens, st, out, vsource, scale, cfg) -> None:
    """Stage B for one layer: split-K decode over st.page_table + LSE merge."""
    sparse_paged_decode_batched(q, kv_cache, block_table, seq_lens, st, out, vsource,
                                scale=scale)


def resolve_selection():
    """(StateClass, derive_fn, select_fn, graph_safe) -- always the HIP path."""
    _lib.load()
    return Rki4State, derive_page_params, _rki4_select_adapter, True
