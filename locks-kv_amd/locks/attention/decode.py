"""Stage B: split-K sparse paged decode + LSE merge on the MI355X kernels.

Call contract of the reference (src/locks/attention/decode.py:130-156,
:328-387): partials m/l (R, n_kv, split, G) and acc (R, n_kv, split, G, D)
fp32 live on the state; pps = max(cdiv(page_cnt, split), pps_min) is derived
on device; ``out`` (T, H, d) rows [0, n_req) are written in place; no host
sync, no allocation.  K comes from the resident paged cache; V through the
V-source seam (only the resident source exists in this build).
"""
from __future__ import annotations

import ctypes

import math

import torch

from .. import _lib

MAX_SPLIT = 512


def _split_kv(kv_cache: torch.Tensor):
    """(K, V) views (num_blocks, page, n_kv, d) for either vLLM cache layout
    ((NB, 2, page, n_kv, d) or (2, NB, page, n_kv, d)); decode.py:64-73."""
    if kv_cache.shape[0] == 2 and kv_cache.shape[1] != 2:
        return kv_cache[0], kv_cache[1]
    if kv_cache.shape[1] == 1:
        return kv_cache.select(1, 0), None
    return kv_cache.select(1, 0), kv_cache.select(1, 1)


class ResidentVSource:
    """V = the resident engine V half of kv_cache (V_SRC=0, decode.py:76-101)."""

    SRC_ID = 0

    def __init__(self, kv_cache: torch.Tensor):
        _, v = _split_kv(kv_cache)
        if v is None:
            raise ValueError("ResidentVSource requires a resident V half; this cache is "
                             "K-only: decode it with the DRAM tier's source "
                             "(locks.tier.TierVSource, mem variants)")
        self._v = v

    def args(self):
        v = self._v
        return v, v.stride(0), v.stride(1), v.stride(2)


COUNTER_STRIDE = 64          # ints between rows' arrival counters (LOCKS_DECODE_COUNTER_STRIDE)
# False (default): the split kernel, then one merge workgroup per query head
# (measured faster per step: 1.306 vs 1.321 ms Llama 128K, 2.529 vs 2.612 ms
# GLM 1M -- the fused form merges a whole row's partials through one CU);
# True: one launch whose last split per row merges the row
FUSED_MERGE = False
PPS_MIN_OVERRIDE = None        # set by bench sweeps; None = the table below


def _pps_min(n_req: int, n_kv: int = 8) -> int:
    """Minimum pages per split workgroup (4 waves, 1-2 pages each at bs=1):
    amortises the q load, the 4-wave LDS merge and the partial store.
    Measured on MI355X at 128 attended pages per row: the best keeps ~256
    split workgroups, i.e. rows / 2 pages per split (at least 4) for rows =
    n_req x n_kv.  Steps at pps_min 16 / 8 / 4: GLM ragged batch of 4 (8
    rows) 1.907 / 1.853 / 1.846 ms, GLM 8 x 64K (16 rows) 1.765 / 1.733 /
    1.801, Llama 4 requests (32 rows) 2.108 / 2.168 / 2.268; bs = 1: Llama
    (8 rows) 4, GLM 1M (2 rows) at 8 / 4 / 2: 2.089-2.093 / 2.048-2.073 /
    2.071-2.084.  From 16 requests 32 (Llama 16 x 32K: 2.88-2.90 ms against
    2.89-2.99 at 16)."""
    if PPS_MIN_OVERRIDE:
        return int(PPS_MIN_OVERRIDE)
    if n_req >= 16:
        return 32
    half = max(1, -(-int(n_req) * int(n_kv) // 2))
    return min(16, max(4, 1 << (half - 1).bit_length()))


def _adaptive_split(max_reqs: int, max_pages: int, budget: float, hard_cap: int) -> int:
    """Allocation-time split count: about the number of active splits the
    expected selection needs at low batch (decode.py:103-127), capped."""
    if int(max_reqs) > 4:
        return min(hard_cap, MAX_SPLIT)
    pps = _pps_min(int(max_reqs))
    est = math.ceil(1.5 * float(budget) * int(max_pages) / max(1, pps))
    p2 = 1 << max(0, (max(1, est) - 1).bit_length())
    return int(min(hard_cap, MAX_SPLIT, max(16, p2)))


def ensure_stage_b_buffers(st, device, split: int) -> None:
    """Allocate the split-K partials on the state once (outside any graph)."""
    if getattr(st, "m_part", None) is not None:
        return
    split = int(min(split, MAX_SPLIT))
    R, n_kv, G, D = st.max_reqs, st.n_kv, st.G, st.D
    st.split = split
    st.m_part = torch.empty(R, n_kv, split, G, device=device, dtype=torch.float32)
    st.l_part = torch.empty(R, n_kv, split, G, device=device, dtype=torch.float32)
    st.acc_part = torch.empty(R, n_kv, split, G, D, device=device, dtype=torch.float32)
    # arrival counts of the fused decode; every call leaves them at zero
    st.dec_counters = torch.zeros(R, n_kv, COUNTER_STRIDE, device=device, dtype=torch.int32)


def decode_splitk(q, k, v, block_table, seq_lens, page_table, page_cnt, m_part, l_part,
                  acc_part, *, n_req: int, G: int, split: int, pps_min: int,
                  scale: float, max_cnt: int = 0) -> None:
    """Launch the split kernel on explicit tensors.  k, v: (NB, page, n_kv, d)
    views; page_table (R, n_kv, MP) i32; page_cnt (R, n_kv) i32."""
    NB, page, n_kv, d = k.shape
    lib = _lib.load()
    _lib.check(lib.locks_decode_splitk(
        _lib.ptr(q), q.stride(0), q.stride(1),
        _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _lib.ptr(v), v.stride(0), v.stride(1), v.stride(2), int(NB),
        _lib.ptr(block_table), block_table.stride(0), int(block_table.shape[1]),
        _lib.ptr(page_table), page_table.stride(0), page_table.stride(1),
        int(page_table.shape[2]), _lib.ptr(page_cnt), page_cnt.stride(0), _lib.ptr(seq_lens),
        _lib.ptr(m_part), _lib.ptr(l_part), _lib.ptr(acc_part), int(n_req), int(n_kv), int(G),
        int(d), int(page), int(split), int(pps_min), int(max_cnt), float(scale),
        _lib.stream_ptr(q.device)), "decode_splitk")


def decode_splitk_tier(q, k, v, block_table, seq_lens, page_table, page_cnt, m_part, l_part,
                       acc_part, tier_src, *, n_req: int, G: int, split: int, pps_min: int,
                       scale: float, max_cnt: int = 0) -> None:
    """The split kernel with V (and, for mem-kv, K) from the DRAM tier
    (``locks.tier.TierVSource.tier_src()``; attention/decode_cuda.py:178-222).
    k, v: (NB, page, n_kv, d) views of the paged cache; v is never read and
    may be any view of k's shape when the cache holds no V half."""
    NB, page, n_kv, d = k.shape
    ts = tier_src
    if (ts.n_kv, ts.page, ts.head_dim, ts.num_blocks) != (n_kv, page, d, NB) \
            or not 0 <= ts.layer < ts.num_layers:
        raise ValueError(f"tier laid out for n_kv {ts.n_kv} / page {ts.page} / head_dim {ts.head_dim} / "
                         f"{ts.num_blocks} blocks, layer {ts.layer} of {ts.num_layers}; the cache is "
                         f"n_kv {n_kv} / page {page} / head_dim {d} / {NB} blocks")
    lib = _lib.load()
    _lib.check(lib.locks_decode_splitk_tier(
        _lib.ptr(q), q.stride(0), q.stride(1),
        _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _lib.ptr(v), v.stride(0), v.stride(1), v.stride(2), int(NB),
        _lib.ptr(block_table), block_table.stride(0), int(block_table.shape[1]),
        _lib.ptr(page_table), page_table.stride(0), page_table.stride(1),
        int(page_table.shape[2]), _lib.ptr(page_cnt), page_cnt.stride(0), _lib.ptr(seq_lens),
        _lib.ptr(m_part), _lib.ptr(l_part), _lib.ptr(acc_part), int(n_req), int(n_kv), int(G),
        int(d), int(page), int(split), int(pps_min), int(max_cnt), float(scale),
        ctypes.addressof(tier_src), _lib.stream_ptr(q.device)), "decode_splitk_tier")


def _check_out(out) -> None:
    """The kernels write 4-element runs along the last dim of ``out``."""
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out must be bf16 or fp32, got {out.dtype}")
    if out.dim() != 3 or out.stride(-1) != 1:
        raise TypeError(f"out must be (n_req, heads, d) with a contiguous last dim, got shape "
                        f"{tuple(out.shape)} strides {tuple(out.stride())}")


def decode_fused(q, k, v, block_table, seq_lens, page_table, page_cnt, m_part, l_part,
                 acc_part, counters, out, *, n_req: int, G: int, split: int, pps_min: int,
                 scale: float, max_cnt: int = 0) -> None:
    """Split kernel whose last-arriving split of each (request, kv head) row
    merges the row into ``out`` (one launch).  ``counters`` (R, n_kv,
    COUNTER_STRIDE) i32 must be zero on the first call; each call leaves it
    zero."""
    if counters.numel() < int(n_req) * k.shape[2] * COUNTER_STRIDE:
        raise ValueError(f"counters needs n_req * n_kv * {COUNTER_STRIDE} int32 entries")
    _check_out(out)
    NB, page, n_kv, d = k.shape
    lib = _lib.load()
    _lib.check(lib.locks_decode_fused(
        _lib.ptr(q), q.stride(0), q.stride(1),
        _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _lib.ptr(v), v.stride(0), v.stride(1), v.stride(2), int(NB),
        _lib.ptr(block_table), block_table.stride(0), int(block_table.shape[1]),
        _lib.ptr(page_table), page_table.stride(0), page_table.stride(1),
        int(page_table.shape[2]), _lib.ptr(page_cnt), page_cnt.stride(0), _lib.ptr(seq_lens),
        _lib.ptr(m_part), _lib.ptr(l_part), _lib.ptr(acc_part), _lib.ptr(counters),
        _lib.ptr(out), out.stride(0), out.stride(1), 1 if out.dtype == torch.float32 else 0,
        int(n_req), int(n_kv), int(G), int(d), int(page), int(split), int(pps_min),
        int(max_cnt), float(scale), _lib.stream_ptr(q.device)), "decode_fused")


def decode_fused_noalloc(q, k, v, block_table, seq_lens, page_table, page_cnt, out, *,
                         n_req: int, G: int, split: int, pps_min: int, scale: float,
                         max_cnt: int = 0) -> None:
    """decode_fused with its split partials and arrival counters in the
    library's fixed per-GPU scratch (LOCKS_NOALLOC_SCRATCH_BYTES): no buffer
    arguments, nothing allocated.  Calls overlapping on one GPU race."""
    _check_out(out)
    NB, page, n_kv, d = k.shape
    lib = _lib.load()
    _lib.check(lib.locks_decode_fused_noalloc(
        _lib.ptr(q), q.stride(0), q.stride(1),
        _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _lib.ptr(v), v.stride(0), v.stride(1), v.stride(2), int(NB),
        _lib.ptr(block_table), block_table.stride(0), int(block_table.shape[1]),
        _lib.ptr(page_table), page_table.stride(0), page_table.stride(1),
        int(page_table.shape[2]), _lib.ptr(page_cnt), page_cnt.stride(0), _lib.ptr(seq_lens),
        _lib.ptr(out), out.stride(0), out.stride(1), 1 if out.dtype == torch.float32 else 0,
        int(n_req), int(n_kv), int(G), int(d), int(page), int(split), int(pps_min),
        int(max_cnt), float(scale), _lib.stream_ptr(q.device)), "decode_fused_noalloc")


def decode_merge(m_part, l_part, acc_part, page_cnt, out, *, n_req: int, n_kv: int, G: int,
                 split: int, pps_min: int, pt_cols: int, max_cnt: int = 0) -> None:
    """LSE merge of the split partials into ``out``; ``pt_cols`` is the page
    table width the split kernel was given (page_cnt is clamped to it)."""
    _check_out(out)
    lib = _lib.load()
    _lib.check(lib.locks_decode_merge(
        _lib.ptr(m_part), _lib.ptr(l_part), _lib.ptr(acc_part), _lib.ptr(page_cnt),
        page_cnt.stride(0), int(pt_cols), _lib.ptr(out), out.stride(0), out.stride(1),
        1 if out.dtype == torch.float32 else 0, int(n_req), int(n_kv), int(G),
        int(acc_part.shape[-1]), int(split), int(pps_min), int(max_cnt),
        _lib.stream_ptr(out.device)),
        "decode_merge")


def decode_dense(q, k, v, block_table, seq_lens, m_part, l_part, acc_part, out, *, n_req: int,
                 G: int, split: int, scale: float) -> None:
    """Dense full-KV decode over every page of each row (the comparator of
    the sparse step): split partials in (R, n_kv, split, G[, d]) buffers,
    then a per-head merge into ``out``."""
    _check_out(out)
    NB, page, n_kv, d = k.shape
    lib = _lib.load()
    _lib.check(lib.locks_decode_dense(
        _lib.ptr(q), q.stride(0), q.stride(1),
        _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _lib.ptr(v), v.stride(0), v.stride(1), v.stride(2), int(NB),
        _lib.ptr(block_table), block_table.stride(0), int(block_table.shape[1]),
        _lib.ptr(seq_lens), _lib.ptr(m_part), _lib.ptr(l_part), _lib.ptr(acc_part),
        _lib.ptr(out), out.stride(0), out.stride(1), 1 if out.dtype == torch.float32 else 0,
        int(n_req), int(n_kv), int(G), int(d), int(page), int(split), float(scale),
        _lib.stream_ptr(q.device)), "decode_dense")


def sparse_paged_decode_batched(q, kv_cache, block_table, seq_lens, st, out,
                                vsource=None, *, scale: float = None) -> None:
    """Batched Stage B (decode.py:328-387): the split kernel + the
    head-parallel merge, or (FUSED_MERGE) one launch whose last split per row
    merges it."""
    if scale is None:
        scale = st.scale
    n_req = seq_lens.shape[0]
    k, _ = _split_kv(kv_cache)
    if vsource is None:
        vsource = ResidentVSource(kv_cache)
    pps = _pps_min(n_req, st.n_kv)
    mc = page_cnt_bound(st)
    if vsource.SRC_ID == 1:
        # DRAM tier (decode_cuda.py:1301-1314): split kernel with the tier's
        # source select, then the same merge
        _, v_res = _split_kv(kv_cache)
        decode_splitk_tier(q, k, v_res if v_res is not None else k, block_table, seq_lens,
                           st.page_table, st.page_cnt, st.m_part, st.l_part, st.acc_part,
                           vsource.tier_src(), n_req=n_req, G=st.G, split=st.split,
                           pps_min=pps, scale=scale, max_cnt=mc)
        decode_merge(st.m_part, st.l_part, st.acc_part, st.page_cnt, out, n_req=n_req,
                     n_kv=st.n_kv, G=st.G, split=st.split, pps_min=pps,
                     pt_cols=st.page_table.shape[2], max_cnt=mc)
        return
    if vsource.SRC_ID != 0:
        raise NotImplementedError(f"V source {vsource.SRC_ID} is not built (0 = resident, 1 = DRAM tier)")
    v = vsource.args()[0]
    if FUSED_MERGE:
        decode_fused(q, k, v, block_table, seq_lens, st.page_table, st.page_cnt, st.m_part,
                     st.l_part, st.acc_part, st.dec_counters, out, n_req=n_req, G=st.G,
                     split=st.split, pps_min=pps, scale=scale, max_cnt=mc)
        return
    decode_splitk(q, k, v, block_table, seq_lens, st.page_table, st.page_cnt, st.m_part,
                  st.l_part, st.acc_part, n_req=n_req, G=st.G, split=st.split,
                  pps_min=pps, scale=scale, max_cnt=mc)
    decode_merge(st.m_part, st.l_part, st.acc_part, st.page_cnt, out, n_req=n_req,
                 n_kv=st.n_kv, G=st.G, split=st.split, pps_min=pps,
                 pt_cols=st.page_table.shape[2], max_cnt=mc)


def page_cnt_bound(st) -> int:
    """Upper bound of any row's page_cnt under the state's budget: b_max
    selected pages plus the sink and window pages (a keep-all row has at most
    sink + 1 + window pages, and b >= 1).  Sizes the decode grid."""
    return int(st.b_max) + int(st.sink_pages) + int(st.window_pages)
