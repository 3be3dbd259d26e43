"""MLA page selection on the MI355X kernels -- the entry the LOCKS MLA
backend forwards to (reference: selection/mla_select.py:111-130
mla_select_pages, backend/mla_attn.py:126-164).

The page score is the reference's max-union over ALL query heads of
(q_c . khat + q_rope . k_rope) * scale (selection/mla_score_torch.py:27-48),
computed from the latent rki4 summary; the keep rule is topb_middle
(sink + recent window forced inside the budget, top-scored middle pages,
:51-73), served by the GQA exact top-b with one "head" and the max combine.
Every entry launches on the current stream, never synchronizes the host and
never allocates.
"""
from __future__ import annotations

import torch

from .. import _lib


def _check_i32(name, t):
    if t.dtype != torch.int32 or not t.is_cuda:
        raise TypeError(f"{name} must be a device int32 tensor, got {t.dtype} on {t.device}")


def _split_cache(kv_cache):
    """(num_blocks, page, 576) bf16 latent cache -> (tensor, block stride, token stride)."""
    if kv_cache.dtype != torch.bfloat16 or kv_cache.dim() != 3 or kv_cache.stride(-1) != 1:
        raise TypeError("MLA cache must be bf16 (num_blocks, page, kv_lora_rank + rope_dim), "
                        "contiguous in the last dim")
    return kv_cache, kv_cache.stride(0), kv_cache.stride(1)


@torch.no_grad()
def mla_build_blocks(st, layer: int, kv_cache, blocks) -> int:
    """(Re)build the latent summaries (and, for an int8-RoPE state, the int8
    RoPE summary) of the listed physical blocks of one layer (the reference's
    per-sequence factor build, mla_select.py:69-108, replaced by the
    block-keyed rki4 latent record)."""
    cache, sb, stt = _split_cache(kv_cache)
    b = blocks.to(device=cache.device, dtype=torch.int32).contiguous()
    n = int(b.numel())
    if n == 0:
        return 0
    v4, vs, c8, cs, mu8, mus, tag = st.layer_state(layer)
    lib = _lib.load()
    _lib.check(lib.locks_build_rki4(
        _lib.ptr(cache), sb, stt, 0, int(min(st.NB, cache.shape[0])), _lib.ptr(b), n, 1, st.D,
        st.page, _lib.ptr(v4), _lib.ptr(vs), _lib.ptr(c8), _lib.ptr(cs), _lib.ptr(mu8),
        _lib.ptr(mus), _lib.rows_arg(st), _lib.ptr(tag), _lib.stream_ptr(cache.device)),
        "build_rki4 (latent)")
    rk8, rks = st.rope_state(layer)
    if rk8 is not None:
        _lib.check(lib.locks_mla_build_rope(
            _lib.ptr(cache), sb, stt, int(min(st.NB, cache.shape[0])), _lib.ptr(b), n, None,
            _lib.ptr(rk8), _lib.ptr(rks), _lib.stream_ptr(cache.device)), "mla_build_rope")
    return n


def mla_derive(st, seq_lens, n_req: int) -> None:
    """n_pages, n_sel_hi = n_pages - window, b = the middle budget."""
    _check_i32("seq_lens", seq_lens)
    lib = _lib.load()
    _lib.check(lib.locks_derive_params(
        _lib.ptr(seq_lens), int(n_req), st.page, st.window_pages, st.sink_pages, st.budget_abs,
        0.5, _lib.ptr(st.n_pages), _lib.ptr(st.n_sel_hi), _lib.ptr(st.b_fix),
        _lib.stream_ptr(seq_lens.device)), "mla derive")


def mla_score_only(st, layer: int, q, kv_cache, block_table, n_req: int, scale: float) -> None:
    """st.score_h[r, 0, 0, p] = page score for the full pages p < n_sel_hi[r]."""
    if q.dtype != torch.bfloat16 or q.stride(-1) != 1:
        raise TypeError("q must be bf16 (T, H, kv_lora_rank + rope_dim) with a contiguous last dim")
    _check_i32("block_table", block_table)
    cache, sb, stt = _split_cache(kv_cache)
    v4, vs, c8, cs, mu8, mus, _tag = st.layer_state(layer)
    rk8, rks = st.rope_state(layer)
    lib = _lib.load()
    _lib.check(lib.locks_mla_score(
        _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(v4), _lib.ptr(vs), _lib.ptr(c8),
        _lib.ptr(cs), _lib.ptr(mu8), _lib.ptr(mus), _lib.ptr(rk8), _lib.ptr(rks),
        _lib.ptr(cache), sb, stt,
        int(min(st.NB, cache.shape[0])), _lib.ptr(block_table), block_table.stride(0),
        int(block_table.shape[1]), _lib.ptr(st.n_sel_hi), _lib.ptr(st.score_h),
        st.score_h.stride(0), int(st.max_pages), int(st.score_chunk), int(n_req), int(q.shape[1]),
        st.D, st.Dr, st.page, float(scale), _lib.stream_ptr(q.device)), "mla_score")


def mla_select_only(st, n_req: int) -> None:
    """Keep rule topb_middle -> st.page_table (R, 1, MP) ascending, st.page_cnt."""
    lib = _lib.load()
    _lib.check(lib.locks_select_nrm_topb(
        _lib.ptr(st.score_h), None, 0, _lib.ptr(st.n_pages), _lib.ptr(st.n_sel_hi),
        _lib.ptr(st.b_fix), _lib.ptr(st.score), _lib.ptr(st.page_table), _lib.ptr(st.page_cnt),
        _lib.ptr(st.sel_ws), st.sel_ws.numel(), int(n_req), 1, 1, int(st.sink_pages),
        int(st.max_pages), 1, int(st.budget_abs), _lib.stream_ptr(st.score.device)), "mla select")


def mla_select_pages(st, layer: int, q, kv_cache, block_table, seq_lens, n_req: int,
                     scale: float) -> None:
    """derive -> latent page score -> topb_middle for every request of the batch."""
    mla_derive(st, seq_lens, n_req)
    mla_score_only(st, layer, q, kv_cache, block_table, n_req, scale)
    mla_select_only(st, n_req)
