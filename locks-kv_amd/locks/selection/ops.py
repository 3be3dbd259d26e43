"""Stage A on the MI355X kernels: derive, score, combine + top-b.

Entry points keep the reference's names and call contracts
(src/locks/selection/select.py:51 derive_page_params,
src/locks/selection/rki4_score_cuda.py:3263 rki4_score_only, :3450
rki4_select_only, :3500 rki4_score_state): they take the caller's tensors,
launch on the current stream, never synchronize the host and never allocate.
"""
from __future__ import annotations

import torch

from .. import _lib


def _check_i32(name, t):
    if t.dtype != torch.int32 or not t.is_cuda:
        raise TypeError(f"{name} must be a device int32 tensor, got {t.dtype} on {t.device}")


def derive_page_params(st, seq_lens, n_req: int) -> None:
    """Refresh st.{n_pages, n_sel_hi, b_fix} for this step (select.py:28-58)."""
    assert n_req <= st.max_reqs
    _check_i32("seq_lens", seq_lens)
    lib = _lib.load()
    _lib.check(lib.locks_derive_params(
        _lib.ptr(seq_lens), int(n_req), st.page, st.window_pages, st.sink_pages,
        st.budget_abs, float(st.budget), _lib.ptr(st.n_pages), _lib.ptr(st.n_sel_hi),
        _lib.ptr(st.b_fix), _lib.stream_ptr(seq_lens.device)), "derive_page_params")


def rki4_score_only(st, layer: int, q, block_table, seq_lens, n_req: int,
                    scale: float) -> None:
    """Write st.score_h (per-head page LSE) for pages [0, n_sel_hi) of each
    request and st.page_max (per-chunk maxima).  seq_lens is unused (every
    scored page is finalized).  A block table narrower than max_pages (the
    engine's memory-profile pass) zeroes score_h instead, as the reference
    does (rki4_score_cuda.py:3332-3353)."""
    if int(block_table.shape[1]) < int(st.max_pages):
        st.score_h.zero_()
        st.page_max.zero_()
        return
    if q.dtype != torch.bfloat16 or q.stride(-1) != 1:
        raise TypeError("q must be bf16 with a contiguous head dim")
    _check_i32("block_table", block_table)
    v4, vs, c8, cs, mu8, mus, _tag = st.layer_state(layer)
    q3 = q.view(q.shape[0], -1, st.d) if q.dim() == 2 else q
    lib = _lib.load()
    _lib.check(lib.locks_score_rki4(
        _lib.ptr(q3), q3.stride(0), q3.stride(1),
        _lib.ptr(v4), _lib.ptr(vs), _lib.ptr(c8), _lib.ptr(cs), _lib.ptr(mu8), _lib.ptr(mus),
        _lib.rows_arg(st), int(st.NB), _lib.ptr(block_table), block_table.stride(0), int(block_table.shape[1]),
        _lib.ptr(st.n_sel_hi), _lib.ptr(st.score_h), int(st.max_pages),
        _lib.ptr(st.page_max), int(st.score_chunk), int(n_req), int(st.n_kv), int(st.G),
        int(st.d), int(st.page), float(scale), _lib.stream_ptr(q.device)), "rki4_score")


def rki4_select_only(st, n_req: int) -> None:
    """GQA combine st.score_h -> st.score and exact top-b -> st.page_table /
    st.page_cnt (fused nrm + top-b, select_cuda.py:493-832, or the "max"
    combine + radix top-b)."""
    lib = _lib.load()
    combine = 0 if st.combine == "nrm" else 1
    _lib.check(lib.locks_select_nrm_topb(
        _lib.ptr(st.score_h), _lib.ptr(st.page_max), int(st.score_chunks),
        _lib.ptr(st.n_pages), _lib.ptr(st.n_sel_hi), _lib.ptr(st.b_fix),
        _lib.ptr(st.score), _lib.ptr(st.page_table), _lib.ptr(st.page_cnt),
        _lib.ptr(st.sel_ws), st.sel_ws.numel(), int(n_req), int(st.n_kv), int(st.G),
        int(st.sink_pages), int(st.max_pages), combine, int(st.b_max),
        _lib.stream_ptr(st.score.device)),
        "select_nrm_topb")


def rki4_score_state(st, layer: int, q, block_table, seq_lens, n_req: int,
                     scale: float) -> None:
    """Score + combine/select for one layer (rki4_score_cuda.py:3500)."""
    rki4_score_only(st, layer, q, block_table, seq_lens, n_req, scale)
    rki4_select_only(st, int(n_req))


def topb_select(st, n_req: int) -> None:
    """No-op kept for call-site compatibility: rki4_select_only already wrote
    page_table / page_cnt (the reference's fused path marks _topb_done the
    same way, select_cuda.py:3740-3744)."""
    return None
