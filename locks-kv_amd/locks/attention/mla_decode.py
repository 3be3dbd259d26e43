"""MLA sparse decode on the MI355X kernels: split-K attention of every query
head over the tokens of the selected latent pages, then the LSE merge.

Replaces the gathered fp32 attention of the reference's
LocksMLAImpl.forward_mqa (backend/mla_attn.py:178-201): softmax over the
selected tokens (position < seq_len) of q . [latent | rope] * scale,
o = P . latent (B, H, kv_lora_rank), lse (B, H).  Partials live on the
MlaState; no host sync, no allocation.
"""
from __future__ import annotations

import torch

from .. import _lib


PPS_MIN_OVERRIDE = None        # set by bench sweeps; None = the table below


def _pps_min(n_req: int) -> int:
    """Minimum pages per split workgroup (the latent page is 18 KB)."""
    if PPS_MIN_OVERRIDE:
        return int(PPS_MIN_OVERRIDE)
    return 4 if n_req <= 4 else 8


def mla_decode(st, q, kv_cache, block_table, seq_lens, n_req: int, scale: float, out,
               lse=None) -> None:
    """out[:n_req] (T, H, 512) bf16 or fp32 and, if given, lse[:n_req] (T, H)
    fp32 from st.page_table / st.page_cnt."""
    if q.dtype != torch.bfloat16 or q.stride(-1) != 1:
        raise TypeError("q must be bf16 (T, H, kv_lora_rank + rope_dim), contiguous last dim")
    if out.dtype not in (torch.bfloat16, torch.float32) or out.stride(-1) != 1:
        raise TypeError("out must be bf16 or fp32 (T, H, kv_lora_rank), contiguous last dim")
    if lse is not None and (lse.dtype != torch.float32 or lse.stride(-1) != 1):
        raise TypeError("lse must be fp32 (T, H)")
    cache = kv_cache
    H = int(q.shape[1])
    pps = _pps_min(n_req)
    lib = _lib.load()
    stream = _lib.stream_ptr(q.device)
    _lib.check(lib.locks_mla_decode_splitk(
        _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(cache), cache.stride(0), cache.stride(1),
        int(min(st.NB, cache.shape[0])), _lib.ptr(block_table), block_table.stride(0),
        int(block_table.shape[1]), _lib.ptr(st.page_table), st.page_table.stride(0),
        int(st.max_pages), _lib.ptr(st.page_cnt), _lib.ptr(seq_lens), _lib.ptr(st.m_part),
        _lib.ptr(st.l_part), _lib.ptr(st.acc_part), int(n_req), H, st.D, st.Dr, st.page,
        int(st.split), pps, float(scale), stream), "mla_decode_splitk")
    _lib.check(lib.locks_mla_decode_merge(
        _lib.ptr(st.m_part), _lib.ptr(st.l_part), _lib.ptr(st.acc_part), _lib.ptr(st.page_cnt),
        int(st.max_pages), _lib.ptr(out), out.stride(0), out.stride(1),
        1 if out.dtype == torch.float32 else 0, _lib.ptr(lse) if lse is not None else None,
        lse.stride(0) if lse is not None else 0, int(n_req), H, st.D, int(st.split), pps,
        stream), "mla_decode_merge")


def mla_decode_dense(q, kv_cache, block_table, seq_lens, m_part, l_part, acc_part, out, *,
                     n_req: int, split: int, scale: float, num_blocks: int, lse=None) -> None:
    """Dense full-cache MLA decode (every page of each row, no page table):
    the comparator of the sparse step.  Partials m/l (R, split, 16) and acc
    (R, split, 16, 512) fp32 (the MlaState layout); out (T, H, 512) bf16 or fp32; lse (T, H) fp32
    or None."""
    if q.dtype != torch.bfloat16 or q.stride(-1) != 1:
        raise TypeError("q must be bf16 (T, H, kv_lora_rank + rope_dim), contiguous last dim")
    if out.dtype not in (torch.bfloat16, torch.float32) or out.stride(-1) != 1:
        raise TypeError("out must be bf16 or fp32 (T, H, kv_lora_rank), contiguous last dim")
    if lse is not None and (lse.dtype != torch.float32 or lse.stride(-1) != 1):
        raise TypeError("lse must be fp32 (T, H)")
    H = int(q.shape[1])
    D = int(out.shape[-1])
    lib = _lib.load()
    _lib.check(lib.locks_mla_decode_dense(
        _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(kv_cache), kv_cache.stride(0),
        kv_cache.stride(1), int(min(num_blocks, kv_cache.shape[0])), _lib.ptr(block_table),
        block_table.stride(0), int(block_table.shape[1]), _lib.ptr(seq_lens), _lib.ptr(m_part),
        _lib.ptr(l_part), _lib.ptr(acc_part), _lib.ptr(out), out.stride(0), out.stride(1),
        1 if out.dtype == torch.float32 else 0, _lib.ptr(lse) if lse is not None else None,
        lse.stride(0) if lse is not None else 0, int(n_req), H, D, int(q.shape[2]) - D,
        int(kv_cache.shape[1]), int(split), float(scale), _lib.stream_ptr(q.device)),
        "mla_decode_dense")
