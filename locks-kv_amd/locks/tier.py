"""DRAM tier data plane: the buffers the split decode reads V (and, for
mem-kv, K) from when a page is not in the paged cache (reference
src/locks/tier/: ``TierVSource`` tier/tier.py:705-784, the decode's
``V_SRC == 1`` seam attention/decode_cuda.py:178-222, its pointer pack
:1043-1070).

Per layer the tier holds
  * a hot buffer (n_kv, S, page, d) bf16 on the GPU with ``page2slot``
    (n_kv, NB) int32 (slot of a (kv head, block), -1 = none; residency.py:329-338);
  * a staging pool (NV, page, n_kv, d) bf16 on the GPU, keyed by ``vbo``
    (NB,) int32 shared over layers (staging block of a block, -1 = none;
    staging.py:334-343);
  * a pinned host pool (L, NB, n_kv, page, d) bf16, read by the GPU through
    its device address (tier.py:57, ``MappedHostVPool``).
The decode picks, per (selected page, kv head): the hot slot when the page is
complete and has one, else the staged block, else the pinned pool.  Which
pages are hot or staged, and when pages move (the reference's LRU residency,
staging lifecycle, leases and copy-engine DMA), is the caller's control
plane; the helpers here only place bytes and set the keys.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _dev_addr(t: torch.Tensor) -> int:
    """Device address of a pinned host tensor (checked by the HIP runtime)."""
    out = ctypes.c_void_p()
    lib = _lib.load()
    _lib.check(lib.locks_host_device_pointer(t.data_ptr(), ctypes.addressof(out)),
               "host_device_pointer")
    return int(out.value)


class TierBuffers:
    """Hot buffer + staging pool + pinned host pool of every layer."""

    def __init__(self, device, *, num_layers: int, num_blocks: int, n_kv: int, head_dim: int,
                 page: int = 16, hot_slots: int, stage_blocks: int, offload_k: bool = False):
        if hot_slots < 1 or stage_blocks < 1:
            raise ValueError("hot_slots and stage_blocks must be >= 1")
        dev = torch.device(device)
        L, NB, S, NV, d = num_layers, num_blocks, hot_slots, stage_blocks, head_dim
        bf16, i32 = torch.bfloat16, torch.int32
        self.L, self.NB, self.n_kv, self.d, self.page, self.S, self.NV = L, NB, n_kv, d, page, S, NV
        self.device, self.offload_k = dev, bool(offload_k)
        self.hot = torch.zeros(L, n_kv, S, page, d, device=dev, dtype=bf16)
        self.page2slot = torch.full((L, n_kv, NB), -1, device=dev, dtype=i32)
        self.v_pool = torch.zeros(L, NV, page, n_kv, d, device=dev, dtype=bf16)
        self.vbo = torch.full((NB,), -1, device=dev, dtype=i32)
        self.pool = torch.zeros(L, NB, n_kv, page, d, dtype=bf16, pin_memory=True)
        self.pool_dev = _dev_addr(self.pool)
        if self.offload_k:
            self.hot_k = torch.zeros_like(self.hot)
            self.k_pool = torch.zeros_like(self.v_pool)
            self.pool_k = torch.zeros(L, NB, n_kv, page, d, dtype=bf16, pin_memory=True)
            self.pool_k_dev = _dev_addr(self.pool_k)

    # ---- byte placement (the control plane decides when) -----------------
    @staticmethod
    def _half(kv_cache, which: int):
        """(NB, page, n_kv, d) view of the K (0) or V (1) half of a
        (NB, 2, page, n_kv, d) cache."""
        return kv_cache[:, which]

    @torch.no_grad()
    def offload(self, layer: int, kv_cache, blocks) -> None:
        """Copy the V (and, with offload_k, K) pages of ``blocks`` of one
        layer's cache into the pinned pool."""
        b = torch.as_tensor(blocks, dtype=torch.long, device=kv_cache.device)
        self.pool[layer, b.cpu()] = self._half(kv_cache, 1)[b].permute(0, 2, 1, 3).cpu()
        if self.offload_k:
            self.pool_k[layer, b.cpu()] = self._half(kv_cache, 0)[b].permute(0, 2, 1, 3).cpu()

    @torch.no_grad()
    def make_hot(self, layer: int, kv_head: int, block: int, slot: int) -> None:
        """Fill hot slot ``slot`` of (layer, kv head) from the pinned pool and
        point (kv head, block) at it."""
        self.hot[layer, kv_head, slot].copy_(self.pool[layer, block, kv_head])
        if self.offload_k:
            self.hot_k[layer, kv_head, slot].copy_(self.pool_k[layer, block, kv_head])
        self.page2slot[layer, kv_head, block] = slot

    def evict(self, layer: int, kv_head: int, block: int) -> None:
        self.page2slot[layer, kv_head, block] = -1

    @torch.no_grad()
    def stage(self, layer: int, kv_cache, block: int, sblock: int) -> None:
        """Copy block ``block`` of one layer's cache (all kv heads) into
        staging block ``sblock`` and key it (vbo is shared over layers)."""
        self.v_pool[layer, sblock].copy_(self._half(kv_cache, 1)[block])
        if self.offload_k:
            self.k_pool[layer, sblock].copy_(self._half(kv_cache, 0)[block])
        self.vbo[block] = sblock

    def unstage(self, block: int) -> None:
        self.vbo[block] = -1

    def vsource(self, layer: int) -> "TierVSource":
        return TierVSource(self, layer)


class TierVSource:
    """The decode's V source for one layer of a tier (tier/tier.py:705-784):
    ``SRC_ID = 1``; ``K_SRC = 1`` when K is offloaded too (mem-kv)."""

    SRC_ID = 1

    def __init__(self, tier: TierBuffers, layer: int):
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
