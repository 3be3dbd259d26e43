"""LOCKS MLA decode -- the host side of the reference's LocksMLAImpl
(backend/mla_attn.py:66-201), which overrides vLLM's MLA ``forward_mqa``:
given the absorbed decode query (q_c | q_rope) and the latent cache, select
pages over the latent summary and attend only to them, returning (o, lse).

vLLM is not installed in this image, so the vLLM subclass itself is not
shipped; ``mla_forward_mqa`` is the body its ``forward_mqa`` calls, with the
reference's semantics: prefill is untouched, rows whose page count fits the
budget attend to every page (topb_middle keep-all), the configured budget
counts the forced sink + recent pages (mla_score_torch.py:63).  One HIP
launch each for derive, score, select, split-K decode and merge -- no host
sync, no allocation, graph-capturable.
"""
from __future__ import annotations

import torch

from ..attention.mla_decode import mla_decode
from ..selection.mla_select import mla_score_only, mla_select_only, mla_select_pages


def mla_layer_index(st, kv_cache) -> int:
    layer_of = getattr(st, "_layer_of", None)
    if layer_of is None:
        raise RuntimeError("locks: MlaState has no kv_cache -> layer map (_layer_of)")
    return layer_of[kv_cache.data_ptr()]


def mla_forward_mqa(q, kv_c_and_k_pe_cache, block_table, seq_lens, st, scale: float, out=None,
                    lse=None, layer: int | None = None, derive: bool = True):
    """q: (B, H, kv_lora_rank + rope_dim) bf16 (or the tuple (q_c, q_rope),
    concatenated as the reference does, mla_attn.py:100-101); the cache
    (num_blocks, page, kv_lora_rank + rope_dim) bf16; seq_lens (B,) int32
    including the current token.  Returns (o (B, H, kv_lora_rank) q.dtype,
    lse (B, H) fp32); ``out`` / ``lse`` are written in place when given.
    ``derive=False`` reuses the page parameters derived earlier in the same
    step (they depend only on seq_lens, so one derive per step suffices)."""
    if isinstance(q, tuple):
        q = torch.cat(q, dim=-1)
    B, H, _ = q.shape
    if layer is None:
        layer = mla_layer_index(st, kv_c_and_k_pe_cache)
    if out is None:
        out = torch.empty(B, H, st.D, dtype=q.dtype, device=q.device)
    if lse is None:
        lse = st.lse[:B, :H]
    if derive:
        mla_select_pages(st, layer, q, kv_c_and_k_pe_cache, block_table, seq_lens, B, scale)
    else:
        mla_score_only(st, layer, q, kv_c_and_k_pe_cache, block_table, B, scale)
        mla_select_only(st, B)
    mla_decode(st, q, kv_c_and_k_pe_cache, block_table, seq_lens, B, scale, out, lse)
    return out, lse
