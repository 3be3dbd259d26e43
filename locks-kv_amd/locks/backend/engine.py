"""Engine-neutral host side of the LOCKS decode path.

One object per model replaces the three places the reference's vLLM
integration spreads this over:

* state allocation, as the metadata builder does once the KV cache exists
  (src/locks/backend/builder.py:658-787): the rki4 state sized by the
  model geometry and the scheduler limits, budget ``cfg.budget`` or 0.1
  when only ``budget_pages`` / a coverage is given, the split-K buffers,
  and the kv-cache pointer -> layer map the select adapter keys on;
* the per-step prologue (builder.py:1100-1136 with the refresh gate
  :1138-1282): summaries refreshed for pages that finalized, then the
  per-request page parameters derived when they can have changed;
* the pure single-token decode forward of the attention impl
  (backend/attn.py:338-378): select the pages of every kv head, then the
  split-K sparse decode with the LSE merge.  Other steps (prefill, mixed
  batches) are the engine's dense attention, as in the reference;
* for the DRAM-tier variants (``mem-v`` / ``mem-kv``) the tier of
  ``locks.tier`` (tier/tier.py:38-302, its decode source :704-784): the
  prologue runs its per-step lifecycle (tier.py:239-301), ``write_kv``
  copies each layer's new V (K) into the staging pool (tier.py:386-392),
  and ``forward`` runs the layer's residency step between selection and the
  decode, which then reads V (K) through ``TierVSource``.

A vLLM-ROCm attention backend calls ``prologue`` from its metadata builder
and ``forward`` from its impl; any other engine can drive it directly.
"""
from __future__ import annotations

import torch

from ..attention.decode import _split_kv, ensure_stage_b_buffers
from ..selection import Rki4State, derive_page_params
from ..tier import Tier
from . import _runtime
from .refresh import RefreshGate


class LocksEngine:
    def __init__(self, cfg, kv_caches, *, num_heads_q: int, num_heads_kv: int, head_dim: int,
                 block_size: int, max_num_seqs: int, max_model_len: int, split: int = 128,
                 max_num_batched_tokens: int = 8192):
        if cfg.mem_summary_cache:
            raise ValueError("locks: mem_summary_cache (summary records in the engine page, K only "
                             "in the tier) is not built; use mem-kv with the K half resident")
        if num_heads_q % num_heads_kv:
            raise ValueError("num_heads_q must be a multiple of num_heads_kv")
        if not kv_caches:
            raise ValueError("kv_caches is empty")
        self.cfg = cfg
        self.kv_caches = list(kv_caches)
        dev = self.kv_caches[0].device
        K0 = _split_kv(self.kv_caches[0])[0]
        page = int(block_size)
        self.st = Rki4State(
            dev, num_layers=len(self.kv_caches), num_blocks=int(K0.shape[0]),
            n_kv=int(num_heads_kv), G=int(num_heads_q // num_heads_kv), head_dim=int(head_dim),
            page=page, max_reqs=int(max_num_seqs), max_pages=-(-int(max_model_len) // page),
            budget=cfg.budget if cfg.budget is not None else 0.1,
            budget_pages=cfg.budget_pages, sink_pages=cfg.sink_pages,
            window_pages=cfg.window_pages, combine=cfg.quad_combine, zsplit=cfg.rki4_zsplit)
        ensure_stage_b_buffers(self.st, dev, split)
        self.st._layer_of = {kv.data_ptr(): i for i, kv in enumerate(self.kv_caches)}
        self.k_layers = [_split_kv(kv)[0] for kv in self.kv_caches]
        self.gate = RefreshGate(page)
        self.tier = None
        if cfg.is_mem:
            self.tier = Tier.from_config(
                cfg, num_layers=len(self.kv_caches), num_blocks=int(K0.shape[0]),
                n_kv=int(num_heads_kv), page=page, d=int(head_dim), max_reqs=int(max_num_seqs),
                max_pages=self.st.max_pages, max_tokens=int(max_num_batched_tokens), device=dev)

    @torch.no_grad()
    def prologue(self, block_table, seq_lens, query_start_loc, n_req: int,
                 seq_lens_cpu=None, query_start_loc_cpu=None):
        """Refresh the summaries and derive the page parameters of this step.

        ``seq_lens`` counts this step's in-flight tokens; the keys of earlier
        steps are in the cache.  Returns the state the layers read."""
        if n_req > self.st.max_reqs:
            raise ValueError(f"n_req {n_req} > max_num_seqs {self.st.max_reqs}")
        if self.tier is not None:
            qsl = query_start_loc
            n_tok = (int(query_start_loc_cpu[n_req]) if query_start_loc_cpu is not None
                     else int(qsl[n_req].item()))
            self.tier.begin_step(block_table, seq_lens, qsl[: n_req + 1], n_req, n_tok)
        need_derive = self.gate.refresh(self.st, self.k_layers, block_table, seq_lens,
                                        query_start_loc, n_req, seq_lens_cpu,
                                        query_start_loc_cpu)
        if need_derive:
            derive_page_params(self.st, seq_lens, n_req)
        return self.st

    @torch.no_grad()
    def forward(self, q, kv_cache, block_table, seq_lens, n_req: int, scale: float, out) -> None:
        """One layer of a pure single-token decode step: ``q`` (n_req, H, d)
        bf16, the layer's kv_cache (its new token already written), ``out``
        (n_req, H, d) written in place."""
        _state, _derive, select_pages, _graph_safe = _runtime.resolve_selection()
        select_pages(q, kv_cache, block_table, seq_lens, self.st, n_req, scale, self.cfg)
        vsource = None
        if self.tier is not None:
            layer = _runtime._layer_index(self.st, kv_cache)
            self.tier.step(layer, self.st.page_table, self.st.page_cnt, block_table, seq_lens, n_req)
            vsource = self.tier.vsource(layer)
        _runtime.decode_dispatch(q, kv_cache, block_table, seq_lens, self.st, out, vsource, scale,
                                 self.cfg)

    @torch.no_grad()
    def write_kv(self, layer: int, key, value) -> None:
        """After the engine wrote this step's K / V (n_tokens, n_kv, d) of one
        layer into its cache: the DRAM tier's copy of them (tier.py:386-392).
        A no-op for the resident variant."""
        if self.tier is not None:
            self.tier.write_kv(layer, value, key)
