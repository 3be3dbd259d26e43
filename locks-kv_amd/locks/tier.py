"""DRAM tier (the mem-v / mem-kv variants): V (and, for mem-kv, K) served
from a bounded GPU hot buffer, a bounded GPU staging pool and a pinned host
pool instead of the paged cache (reference src/locks/tier/: ``Tier``
tier/tier.py:38-302, ``Residency`` residency.py:310-459, ``Staging``
staging.py:280-570, ``TierVSource`` tier.py:704-784, the decode's
``V_SRC == 1`` seam attention/decode_cuda.py:178-222).

Per step (``begin_step``, before the layers, once): pages written this step
lose their hot residency and pool validity; complete staged pages are copied
to the pinned pool and their staging blocks freed; the pages this step writes
get staging blocks and the per-token staging slots.  Per layer: ``write_kv``
scatters the step's V (K) into the staging pool; after selection, ``step``
classifies the selected pages against the hot buffer, installs the misses
into least-recently-used slots and copies their bytes in.  The decode then
reads each selected page from its hot slot (complete page with a slot), else
its staging block, else the pinned pool.  Every stage is a HIP kernel
(csrc/locks_tier.hip); nothing synchronizes the host.

Buffers (all layers):
  * hot (L, n_kv, S, page, d) bf16, page2slot (L, n_kv, NB) i32 (-1 = none),
    slot2page (L, n_kv, S), lru (L, n_kv, S) clocks, clock (L, n_kv),
    pool_valid (L, n_kv, NB) i8 (residency.py:329-366);
  * v_pool (L, NV, page, n_kv, d) bf16 staging, vbo (NB,) staging block of a
    block (-1 = none), v_flushed (NB,), free stack, flush list, per-token
    v_slot_mapping (staging.py:330-356);
  * pool (L, NB, n_kv, page, d) bf16 pinned host memory, read and written by
    the GPU through its device address (pool.py ``MappedHostVPool``).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib


def _dev_addr(t: torch.Tensor) -> int:
    """Device address of a pinned host tensor (checked by the HIP runtime)."""
    out = ctypes.c_void_p()
    lib = _lib.load()
    _lib.check(lib.locks_host_device_pointer(t.data_ptr(), ctypes.addressof(out)),
               "host_device_pointer")
    return int(out.value)


def _i32(name, t):
    if t.dtype != torch.int32 or not t.is_cuda:
        raise TypeError(f"{name} must be a device int32 tensor, got {t.dtype} on {t.device}")


class Tier:
    """Hot buffer + staging pool + pinned pool of every layer, with the
    per-step staging lifecycle and the per-layer exact-LRU residency."""

    def __init__(self, device, *, num_layers: int, num_blocks: int, n_kv: int, head_dim: int,
                 page: int = 16, hot_slots: int, max_reqs: int = 1, max_pages: int = 1,
                 max_tokens: int = 8192, v_blocks: int | None = None,
                 max_flush: int | None = None, offload_k: bool = False):
        if hot_slots < 1:
            raise ValueError("hot_slots must be >= 1")
        dev = torch.device(device)
        L, NB, S, d = num_layers, num_blocks, hot_slots, head_dim
        chunk_pages = -(-int(max_tokens) // page)
        NV = int(v_blocks) if v_blocks else Tier.default_v_blocks(chunk_pages, max_reqs)
        MAXF = int(max_flush) if max_flush else chunk_pages + 2 * max_reqs + 64
        if NV < chunk_pages + max_reqs:
            # staging.py:606-621: one prefill chunk must fit, or V could be lost
            raise ValueError(f"v_blocks {NV} < chunk_pages {chunk_pages} + max_reqs {max_reqs}")
        bf16, i32 = torch.bfloat16, torch.int32
        self.L, self.NB, self.n_kv, self.d, self.page, self.S, self.NV = L, NB, n_kv, d, page, S, NV
        self.R, self.MP, self.max_tokens, self.MAXF = int(max_reqs), int(max_pages), int(max_tokens), MAXF
        self.device, self.offload_k = dev, bool(offload_k)
        # residency
        self.hot = torch.zeros(L, n_kv, S, page, d, device=dev, dtype=bf16)
        self.page2slot = torch.full((L, n_kv, NB), -1, device=dev, dtype=i32)
        self.slot2page = torch.full((L, n_kv, S), -1, device=dev, dtype=i32)
        self.lru = torch.zeros(L, n_kv, S, device=dev, dtype=i32)
        self.clock = torch.zeros(L, n_kv, device=dev, dtype=i32)
        self.pool_valid = torch.zeros(L, n_kv, NB, device=dev, dtype=torch.int8)
        self.FCAP = self.R * self.MP
        self.miss_pages = torch.zeros(self.R, n_kv, self.MP, device=dev, dtype=i32)
        self.miss_cnt = torch.zeros(self.R, n_kv, device=dev, dtype=i32)
        self.victims = torch.zeros(self.R, n_kv, self.MP, device=dev, dtype=i32)
        self.fetch_list = torch.zeros(n_kv, self.FCAP, 2, device=dev, dtype=i32)
        self.fetch_cnt = torch.zeros(n_kv, device=dev, dtype=i32)
        self.res_overflow = torch.zeros(1, device=dev, dtype=i32)
        # staging
        self.v_pool = torch.zeros(L, NV, page, n_kv, d, device=dev, dtype=bf16)
        self.vbo = torch.full((NB,), -1, device=dev, dtype=i32)
        self.v_flushed = torch.zeros(NB, device=dev, dtype=i32)
        self.free_stack = torch.arange(NV, device=dev, dtype=i32)
        self.free_top = torch.full((1,), NV, device=dev, dtype=i32)
        self.flush_list = torch.zeros(MAXF, 2, device=dev, dtype=i32)
        self.flush_cnt = torch.zeros(1, device=dev, dtype=i32)
        self.v_slot_mapping = torch.full((self.max_tokens,), -1, device=dev, dtype=torch.int64)
        self.stg_overflow = torch.zeros(1, device=dev, dtype=i32)
        # pinned pools
        self.pool = torch.zeros(L, NB, n_kv, page, d, dtype=bf16, pin_memory=True)
        self.pool_dev = _dev_addr(self.pool)
        if self.offload_k:
            self.hot_k = torch.zeros_like(self.hot)
            self.k_pool = torch.zeros_like(self.v_pool)
            self.pool_k = torch.zeros(L, NB, n_kv, page, d, dtype=bf16, pin_memory=True)
            self.pool_k_dev = _dev_addr(self.pool_k)

    # ---- sizing (tier.py:139-238, staging.py:284-289) ----------------------
    @staticmethod
    def default_v_blocks(chunk_pages: int, max_reqs: int) -> int:
        """Staging working set: one prefill chunk (collect frees the previous
        chunk before valloc), 25 % margin, per-request partial tails."""
        return chunk_pages + chunk_pages // 4 + 4 * max_reqs + 64

    @staticmethod
    def recommend_hot_slots(budget_frac: float, max_pages: int, *, target_ratio: float = 6.0,
                            sink: int = 1, win: int = 1, floor: int = 64, n_seqs: int = 1,
                            budget_pages: int | None = None) -> int:
        """Hot slots per (layer, kv head) proportional to the selected working
        set: target_ratio x b + sink + window per sequence at bs = 1; with
        several sequences the attended set per sequence; floored, and capped at
        every page of every sequence."""
        selectable = max(1, int(max_pages) - sink - win)
        b = max(1, math.ceil(float(budget_frac) * selectable))
        ns = max(1, int(n_seqs))
        if ns > 1:
            bp = b if (budget_pages is None or int(budget_pages) <= 0) else min(int(budget_pages), selectable)
            s = (bp + sink + win) * ns
        else:
            s = (math.ceil(target_ratio * b) + sink + win) * ns
        s = max(floor, s)
        return int(min(s, max(int(max_pages) * ns, floor)))

    @classmethod
    def from_config(cls, cfg, *, num_layers, num_blocks, n_kv, page, d, max_reqs, max_pages,
                    max_tokens, device) -> "Tier":
        """Tier of a mem variant of ``LocksConfig`` (tier.py:207-237):
        ``hot_slots <= 0`` sizes the hot buffer from the budget."""
        if not cfg.is_mem:
            raise ValueError(f"Tier requires a mem variant, got {cfg.variant!r}")
        hot = cfg.hot_slots
        if hot is None or hot <= 0:
            hot = cls.recommend_hot_slots(
                cfg.budget if cfg.budget is not None else 0.15, max_pages, n_seqs=max_reqs,
                target_ratio=float(cfg.hot_ratio), sink=cfg.sink_pages, win=cfg.window_pages,
                budget_pages=cfg.budget_pages)
        return cls(device, num_layers=num_layers, num_blocks=num_blocks, n_kv=n_kv, head_dim=d,
                   page=page, hot_slots=int(hot), max_reqs=max_reqs, max_pages=max_pages,
                   max_tokens=max_tokens, v_blocks=cfg.v_blocks, offload_k=cfg.offload_k)

    # ---- per step (tier.py:239-301) ----------------------------------------
    @torch.no_grad()
    def begin_step(self, block_table, seq_lens, query_start_loc, n_req: int, n_tokens: int) -> None:
        """Invalidate the pages written this step, then the staging
        lifecycle (flush-latch clear, collect + free, flush copy to the
        pinned pool, staging allocation, token slots).  ``seq_lens`` count
        this step's tokens; ``query_start_loc`` (n_req + 1,) int32."""
        if n_tokens > self.max_tokens:
            raise RuntimeError(f"tier begin_step: {n_tokens} tokens > max_tokens {self.max_tokens}")
        for n, t in (("block_table", block_table), ("seq_lens", seq_lens),
                     ("query_start_loc", query_start_loc)):
            _i32(n, t)
        lib, s = _lib.load(), _lib.stream_ptr(self.device)
        bt = block_table
        _lib.check(lib.locks_tier_invalidate(
            _lib.ptr(bt), bt.stride(0), int(bt.shape[1]), _lib.ptr(seq_lens),
            _lib.ptr(query_start_loc), int(n_req), _lib.ptr(self.page2slot), _lib.ptr(self.slot2page),
            _lib.ptr(self.pool_valid), self.L, self.n_kv, self.NB, self.S, self.page, s),
            "tier_invalidate")
        _lib.check(lib.locks_tier_stage_begin(
            _lib.ptr(bt), bt.stride(0), int(bt.shape[1]), _lib.ptr(seq_lens),
            _lib.ptr(query_start_loc), int(n_req), _lib.ptr(self.vbo), _lib.ptr(self.v_flushed),
            _lib.ptr(self.free_stack), _lib.ptr(self.free_top), _lib.ptr(self.flush_list),
            _lib.ptr(self.flush_cnt), self.MAXF, _lib.ptr(self.v_slot_mapping), self.max_tokens,
            _lib.ptr(self.stg_overflow), self.NB, self.NV, self.page, s), "tier_stage_begin")
        vp = self.v_pool
        kt = self.offload_k
        _lib.check(lib.locks_tier_flush_copy(
            _lib.ptr(self.flush_list), _lib.ptr(self.flush_cnt), self.MAXF, _lib.ptr(vp),
            _lib.ptr(self.k_pool) if kt else 0, vp.stride(0), vp.stride(1), vp.stride(2), vp.stride(3),
            self.pool_dev, self.pool_k_dev if kt else 0, _lib.ptr(self.pool_valid), self.L,
            self.n_kv, self.NB, self.page, self.d, 1 if kt else 0, s), "tier_flush_copy")

    @torch.no_grad()
    def write_kv(self, layer: int, value, key=None, n_tokens: int | None = None) -> None:
        """This step's V (and, mem-kv, K) (n_tokens, n_kv, d) bf16 of one
        layer into its staging pool at the token slots (staging.py:444-460;
        the engine's cache write of the same tokens is unchanged)."""
        n = int(value.shape[0] if n_tokens is None else n_tokens)
        if self.offload_k and key is None:
            raise ValueError("mem-kv: write_kv needs the key")
        vp = self.v_pool[layer]
        kp = self.k_pool[layer] if self.offload_k else None
        k = key if self.offload_k else None
        _lib.check(_lib.load().locks_tier_scatter(
            _lib.ptr(value), value.stride(0), value.stride(1), _lib.ptr(k),
            k.stride(0) if k is not None else 0, k.stride(1) if k is not None else 0, n,
            _lib.ptr(self.v_slot_mapping), _lib.ptr(vp), _lib.ptr(kp), vp.stride(0), vp.stride(1),
            vp.stride(2), self.n_kv, self.d, self.page, self.NV, 1 if self.offload_k else 0,
            _lib.stream_ptr(self.device)), "tier_scatter")

    @torch.no_grad()
    def step(self, layer: int, page_table, page_cnt, block_table, seq_lens, n_req: int) -> None:
        """Residency of one layer after selection (residency.py:421-488):
        plan (hits touched, misses installed into LRU victims) + fetch."""
        if int(page_table.shape[-1]) != self.MP or n_req > self.R:
            raise ValueError(f"page table (.., {int(page_table.shape[-1])}) / n_req {n_req} do not match "
                             f"the tier's max_pages {self.MP} / max_reqs {self.R}")
        lib, s = _lib.load(), _lib.stream_ptr(self.device)
        bt, pt = block_table, page_table
        _lib.check(lib.locks_tier_plan(
            _lib.ptr(pt), pt.stride(0), pt.stride(1), int(pt.shape[2]), _lib.ptr(page_cnt),
            page_cnt.stride(0), _lib.ptr(bt), bt.stride(0), int(bt.shape[1]), _lib.ptr(seq_lens),
            int(n_req), _lib.ptr(self.page2slot[layer]), _lib.ptr(self.slot2page[layer]),
            _lib.ptr(self.lru[layer]), _lib.ptr(self.clock[layer]), _lib.ptr(self.miss_pages),
            _lib.ptr(self.miss_cnt), _lib.ptr(self.victims), _lib.ptr(self.fetch_list),
            _lib.ptr(self.fetch_cnt), self.FCAP, _lib.ptr(self.res_overflow), self.n_kv, self.NB,
            self.S, self.page, s), "tier_plan")
        vp = self.v_pool[layer]
        kt = self.offload_k
        _lib.check(lib.locks_tier_fetch(
            _lib.ptr(self.fetch_list), _lib.ptr(self.fetch_cnt), self.FCAP, _lib.ptr(self.hot[layer]),
            _lib.ptr(self.hot_k[layer]) if kt else 0, self.pool_dev, self.pool_k_dev if kt else 0,
            _lib.ptr(vp), _lib.ptr(self.k_pool[layer]) if kt else 0, vp.stride(0), vp.stride(1),
            vp.stride(2), _lib.ptr(self.vbo), _lib.ptr(self.pool_valid[layer]), int(layer), self.L,
            self.n_kv, self.NB, self.S, self.NV, self.page, self.d, 1 if kt else 0, s), "tier_fetch")

    def vsource(self, layer: int) -> "TierVSource":
        return TierVSource(self, layer)

    # ---- invariants (host-syncing, for tests and debugging) ---------------
    def check_invariants(self) -> None:
        """residency.py:602-765 R1-R3 (page2slot and slot2page mutual
        inverses) and staging.py:572-588 (assigned + free staging blocks
        partition [0, NV)); raises AssertionError."""
        p2s, s2p = self.page2slot.cpu(), self.slot2page.cpu()
        for l in range(self.L):
            for kv in range(self.n_kv):
                pg = s2p[l, kv]
                occ = torch.nonzero(pg >= 0).flatten()
                if pg[occ].unique().numel() != occ.numel():
                    raise AssertionError(f"layer {l} kv {kv}: two slots hold one page")
                if not torch.equal(p2s[l, kv][pg[occ].long()], occ.to(torch.int32)):
                    raise AssertionError(f"layer {l} kv {kv}: slot2page -> page2slot broken")
                adv = torch.nonzero(p2s[l, kv] >= 0).flatten()
                if not torch.equal(pg[p2s[l, kv][adv].long()], adv.to(torch.int32)):
                    raise AssertionError(f"layer {l} kv {kv}: page2slot -> slot2page broken")
        vbo, top = self.vbo.cpu(), int(self.free_top.item())
        assigned = vbo[vbo >= 0]
        free = self.free_stack.cpu()[:top]
        allv = torch.cat([assigned, free])
        if allv.numel() != self.NV or allv.unique().numel() != self.NV:
            raise AssertionError(f"staging blocks: {assigned.numel()} assigned + {top} free != NV {self.NV}")

    # ---- manual placement (data-plane tests; bypasses the lifecycle) -------
    @staticmethod
    def _half(kv_cache, which: int):
        """(NB, page, n_kv, d) view of the K (0) or V (1) half of a
        (NB, 2, page, n_kv, d) cache."""
        return kv_cache[:, which]

    @torch.no_grad()
    def offload(self, layer: int, kv_cache, blocks) -> None:
        """Copy the V (and K) pages of ``blocks`` of one layer's cache into
        the pinned pool and mark them pool-valid."""
        b = torch.as_tensor(blocks, dtype=torch.long, device=kv_cache.device)
        self.pool[layer, b.cpu()] = self._half(kv_cache, 1)[b].permute(0, 2, 1, 3).cpu()
        if self.offload_k:
            self.pool_k[layer, b.cpu()] = self._half(kv_cache, 0)[b].permute(0, 2, 1, 3).cpu()
        self.pool_valid[layer][:, b] = 1

    @torch.no_grad()
    def make_hot(self, layer: int, kv_head: int, block: int, slot: int) -> None:
        """Fill hot slot ``slot`` of (layer, kv head) from the pinned pool and
        point (kv head, block) at it, unmapping the slot's previous page."""
        old = int(self.slot2page[layer, kv_head, slot])
        if old >= 0:
            self.page2slot[layer, kv_head, old] = -1
        self.hot[layer, kv_head, slot].copy_(self.pool[layer, block, kv_head])
        if self.offload_k:
            self.hot_k[layer, kv_head, slot].copy_(self.pool_k[layer, block, kv_head])
        self.page2slot[layer, kv_head, block] = slot
        self.slot2page[layer, kv_head, slot] = block

    def evict(self, layer: int, kv_head: int, block: int) -> None:
        slot = int(self.page2slot[layer, kv_head, block])
        if slot >= 0:
            self.slot2page[layer, kv_head, slot] = -1
        self.page2slot[layer, kv_head, block] = -1

    @torch.no_grad()
    def stage(self, kv_caches, block: int, sblock: int) -> None:
        """Copy block ``block`` of every layer's cache (``kv_caches``: one
        (NB, 2, page, n_kv, d) cache per layer) into staging block ``sblock``
        and key it; ``vbo`` is shared by the layers, so all are staged."""
        if len(kv_caches) != self.L:
            raise ValueError(f"stage needs all {self.L} layers' caches, got {len(kv_caches)}")
        for layer, kv in enumerate(kv_caches):
            self.v_pool[layer, sblock].copy_(self._half(kv, 1)[block])
            if self.offload_k:
                self.k_pool[layer, sblock].copy_(self._half(kv, 0)[block])
        self.vbo[block] = sblock

    def unstage(self, block: int) -> None:
        self.vbo[block] = -1


class TierVSource:
    """The decode's V source for one layer of a tier (tier/tier.py:705-784):
    ``SRC_ID = 1``; ``K_SRC = 1`` when K is offloaded too (mem-kv)."""

    SRC_ID = 1

    def __init__(self, tier: Tier, layer: int):
        if not 0 <= layer < tier.L:
            raise ValueError(f"layer {layer} outside [0, {tier.L})")
        self._t, self._l = tier, int(layer)
        self.K_SRC = 1 if tier.offload_k else 0

    def args(self):
        """Staging V pool of the layer and its element strides (tier.py:732-736)."""
        vp = self._t.v_pool[self._l]
        return vp, vp.stride(0), vp.stride(1), vp.stride(2)

    def k_args(self):
        kp = self._t.k_pool[self._l]
        return kp, kp.stride(0), kp.stride(1), kp.stride(2)

    def k_tier_ptrs(self):
        t = self._t
        return t.hot_k[self._l], t.pool_k

    def union(self) -> dict:
        """Pointer union of the layer (tier.py:765-784)."""
        t, l = self._t, self._l
        return dict(lidx=l, NB=t.NB, S=t.S, n_kv=t.n_kv, page=t.page, d=t.d, hot=t.hot[l],
                    page2slot=t.page2slot[l], v_pool=t.v_pool[l], vbo=t.vbo, pool=t.pool)

    def tier_src(self) -> "_lib.TierSrc":
        """The C ABI's locks_tier_src of this layer (attention/decode_cuda.py:1043-1070)."""
        t, l = self._t, self._l
        vp = t.v_pool[l]
        ts = _lib.TierSrc()
        ts.hot_v, ts.stage_v, ts.pool_v = t.hot[l].data_ptr(), vp.data_ptr(), t.pool_dev
        if t.offload_k:
            kp = t.k_pool[l]
            if kp.stride() != vp.stride():
                raise ValueError("the K staging pool must share the V staging pool's strides")
            ts.hot_k, ts.stage_k, ts.pool_k = t.hot_k[l].data_ptr(), kp.data_ptr(), t.pool_k_dev
        ts.page2slot, ts.vbo = t.page2slot[l].data_ptr(), t.vbo.data_ptr()
        ts.stage_stride_block, ts.stage_stride_tok, ts.stage_stride_head = vp.stride(0), vp.stride(1), vp.stride(2)
        ts.num_blocks, ts.hot_slots, ts.stage_blocks = t.NB, t.S, t.NV
        ts.layer, ts.k_tier = l, 1 if t.offload_k else 0
        ts.n_kv, ts.page, ts.head_dim, ts.num_layers = t.n_kv, t.page, t.d, t.L
        return ts
